"""Helpers of the GPU parity tests: run each C-ABI entry point on device tensors and bring the results back."""
from __future__ import annotations

import numpy as np
import torch

from cdna4_sage import _capi
from oracle import sage_oracle as orc

DT = {torch.bfloat16: _capi.DTYPE_BF16, torch.float16: _capi.DTYPE_F16}


def bsh(t: torch.Tensor, layout: str):
    return (t.stride(0), t.stride(2), t.stride(1)) if layout == "HND" else (t.stride(0), t.stride(1), t.stride(2))


def stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def run_quant_q(q: torch.Tensor, layout="HND", qs_mul=1.0):
    dev = q.device
    if layout == "HND":
        B, H, S, D = q.shape
    else:
        B, S, H, D = q.shape
    dl = _capi.layout_dim(D)
    q8 = torch.empty(B, H, S, dl, dtype=torch.int8, device=dev)
    qs = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    _capi.call("sage_quant_q", q.data_ptr(), *bsh(q, layout), B, H, S, D, DT[q.dtype], qs_mul, q8.data_ptr(),
               qs.data_ptr(), stream(dev))
    torch.cuda.synchronize(dev)
    return q8.cpu().numpy(), qs.cpu().numpy()


def run_quant_kv(k: torch.Tensor, v: torch.Tensor, layout="HND"):
    dev = k.device
    if layout == "HND":
        B, Hkv, S, D = k.shape
    else:
        B, S, Hkv, D = k.shape
    skp = _capi.kv_pad(S)
    dl = _capi.layout_dim(D)
    vs = torch.empty(B, Hkv, dl, dtype=torch.float32, device=dev)
    k8 = torch.empty(B, Hkv, skp, dl, dtype=torch.int8, device=dev)
    ks = torch.empty(B, Hkv, skp // 32, dtype=torch.float32, device=dev)
    v8t = torch.empty(B, Hkv, dl, skp, dtype=torch.uint8, device=dev)
    st = stream(dev)
    _capi.call("sage_v_amax", v.data_ptr(), *bsh(v, layout), B, Hkv, S, D, DT[v.dtype], vs.data_ptr(), st)
    _capi.call("sage_quant_kv", k.data_ptr(), *bsh(k, layout), v.data_ptr(), *bsh(v, layout), B, Hkv, S, D,
               DT[k.dtype], vs.data_ptr(), k8.data_ptr(), ks.data_ptr(), v8t.data_ptr(), st)
    torch.cuda.synchronize(dev)
    return k8.cpu().numpy(), ks.cpu().numpy(), v8t.cpu().numpy(), vs.cpu().numpy()


def hnd_np(t: torch.Tensor, layout="HND") -> np.ndarray:
    """float32 numpy copy in HND layout."""
    t = t if layout == "HND" else t.transpose(1, 2)
    return t.float().cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float((a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum()))


def fp32_cos_head(q, k, v, out, causal, chunk=4096):
    """Cosine between one head's output and float32 attention computed on the GPU in row chunks (q [Sq, D], k / v
    [Skv, D] float32 device tensors, out [Sq, D])."""
    sq, skv, d = q.shape[0], k.shape[0], q.shape[1]
    kt = k.t().contiguous()
    num = den_a = den_b = 0.0
    for r0 in range(0, sq, chunk):
        r1 = min(sq, r0 + chunk)
        s = torch.matmul(q[r0:r1], kt) * (d ** -0.5)
        if causal:
            last = torch.arange(r0, r1, device=q.device)[:, None] + (skv - sq)
            s = s.masked_fill(torch.arange(skv, device=q.device)[None, :] > last, float("-inf"))
        ref = torch.matmul(torch.softmax(s, dim=-1), v)
        o = out[r0:r1].float()
        num += float((o * ref).sum())
        den_a += float((o * o).sum())
        den_b += float((ref * ref).sum())
    return num / (den_a * den_b) ** 0.5


def kv_split(dev, B, H, Sq, Skv, D, causal, heads=None):
    """The emulation's ``kv_split`` argument that follows the attention kernel's plan on `dev` (None when the plan
    splits nothing).  ``heads``: indices, in the full problem of H heads, of the heads an emulated sample holds."""
    n_full, chunks, _ = _capi.attn_plan(torch.device(dev).index or 0, B, H, Sq, Skv, D, bool(causal))
    if chunks <= 1:
        return None
    return chunks, orc.split_rows(B, H, Sq, n_full, heads=heads)


def unpad(a: np.ndarray, d: int, axis: int = -1) -> np.ndarray:
    """The first d channels of a layout array along `axis`; asserts the padding channels (head_dim 96 is stored as
    128 channels) are zero."""
    a = np.moveaxis(np.asarray(a), axis, -1)
    assert not np.any(a[..., d:]), "padding channels must be zero"
    return np.moveaxis(a[..., :d], -1, axis)


WALK_MAX_ABS = 2e-2


def assert_near_walk(got, walk, ref):
    """Rows of split query tiles against the reference's own walk of every key in one online softmax
    (kernel_build/make_sage_r2.py:141-253; the emulation without ``kv_split``): max-abs 2e-2, or, where outlier
    channels make the outputs large (x10 V channels: outputs up to ~50, whose bf16 step alone is 0.25), the walk's
    own largest distance to float64 attention ``ref`` on the same rows.  Returns the largest difference."""
    gap = float(np.abs(np.asarray(got, np.float64) - walk).max())
    own = float(np.abs(np.asarray(walk, np.float64) - ref).max())
    assert gap <= max(WALK_MAX_ABS, own), (gap, own)
    return gap


def underflow_split_inputs(seed=3):
    """One head (Sq 128, Skv 1024, head dim 128, bf16 values as float32 [1, 1, S, 128]) whose query rows all point
    along one direction u: key 0 is 20 u, every other key -16 u (plus noise), the rows 30 u times 0.9 to 1.1.  Key 0
    leads every other key by ~124 to ~152 in the exponent (log2 units), so a split range that starts from the
    running max after key tile 0 holds only probabilities of 2^-124 to 2^-152: its l falls below 2^-128, or to 0,
    and every E4M3 byte of its P is 0.  The output is V of key 0."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(128, generator=g)
    u = u / u.norm()
    f = 0.9 + 0.2 * torch.rand(128, 1, generator=g)
    q = 30.0 * f * u + 0.02 * torch.randn(128, 128, generator=g)
    k = -16.0 * u + 0.02 * torch.randn(1024, 128, generator=g)
    k[0] = 20.0 * u
    v = torch.randn(1024, 128, generator=g)
    return [t[None, None].to(torch.bfloat16).float().numpy() for t in (q, k, v)]
