"""int8 QK / fp8 PV attention for MI355X (gfx950): quantize Q, K, V and run the CDNA4 kernel.

Mirrors src/rdna4_sage/_attention.py (same names, arguments and error behaviour) with the launch boundary moved into
libsage_capi.so: one C call runs V amax, the Q quantizer, the K/V quantizer and the attention kernel on torch's
current stream.  Intermediates are torch-owned (caching allocator), as in the reference (_attention.py:115-133).
"""
from __future__ import annotations

import functools
import json
import math
from pathlib import Path

import torch

from . import _capi

_MANIFEST_PATH = Path(__file__).resolve().parent / "manifest.json"
_MANIFEST = json.loads(_MANIFEST_PATH.read_text())
KV_BLOCK = _MANIFEST["kv_block"]            # keys per K scale (reference: kernels/manifest.json "kv_block")
HEAD_DIMS = tuple(_MANIFEST["head_dims"])
LSE_HEAD_DIMS = tuple(_MANIFEST["lse"]["head_dims"])   # the LSE kernel; other head dims use the torch formula
ARCHS = (_MANIFEST["arch"],)
DTYPES = {torch.bfloat16: _capi.DTYPE_BF16, torch.float16: _capi.DTYPE_F16}
_I32_MAX = 2**31 - 1

_arch_cache = {}


class Unsupported(Exception):
    """The inputs fall outside what the gfx950 kernels handle; use another attention backend."""


def device_arch(device: torch.device) -> str:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _arch_cache:
        _arch_cache[idx] = torch.cuda.get_device_properties(idx).gcnArchName.split(":")[0]
    return _arch_cache[idx]


def _bsh(t: torch.Tensor, layout: str):
    """(batch, seq, head) element strides.  The quantizers load 16-byte vectors, so the base must be 16-byte aligned
    and the strides multiples of 8 elements; anything else is copied to a new contiguous tensor (reference:
    _attention.py:59-67).  .contiguous() alone would keep an already contiguous tensor on a misaligned base."""
    s = t.stride()
    if s[3] != 1 or t.data_ptr() % 16 or s[0] % 8 or s[1] % 8 or s[2] % 8:
        t = t.clone(memory_format=torch.contiguous_format)
        s = t.stride()
    return t, ((s[0], s[2], s[1]) if layout == "HND" else s[:3])


def check_supported(q, k, v, layout, is_causal=False):
    """Raise Unsupported with the reason if the gfx950 kernels cannot run these inputs (reference:
    _attention.py:70-94, with the architecture set {gfx950} and head dims {64, 128})."""
    if layout not in ("HND", "NHD"):
        raise Unsupported(f"layout {layout!r}")
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise Unsupported("tensors must be on one ROCm GPU")
    if q.dtype not in DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise Unsupported(f"dtype {q.dtype}/{k.dtype}/{v.dtype} (fp16 or bf16 required)")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise Unsupported("4D tensors required")
    arch = device_arch(q.device)
    if arch not in ARCHS:
        raise Unsupported(f"GPU {arch} is not CDNA4 (kernels built for {', '.join(ARCHS)} only)")
    hd = q.shape[-1]
    if hd not in HEAD_DIMS or k.shape[-1] != hd or v.shape[-1] != hd:
        raise Unsupported(f"head_dim {hd} (supported {HEAD_DIMS})")
    h_ax, s_ax = (1, 2) if layout == "HND" else (2, 1)
    if q.shape[0] != k.shape[0] or k.shape[0] != v.shape[0] or k.shape[h_ax] != v.shape[h_ax] or k.shape[s_ax] != v.shape[s_ax]:
        raise Unsupported("q/k/v batch, k/v heads and k/v lengths must match")
    if max(q.numel(), k.numel()) > _I32_MAX or k.numel() == 0 or q.numel() == 0:
        raise Unsupported("tensor too large for 32-bit indexing or empty")
    if q.shape[h_ax] % k.shape[h_ax]:
        raise Unsupported(f"heads {q.shape[h_ax]} not a multiple of kv heads {k.shape[h_ax]}")
    if is_causal and q.shape[s_ax] > k.shape[s_ax]:
        raise Unsupported("causal attention needs q_len <= kv_len (bottom-right aligned)")


def qs_fold_factor(sm_scale, head_dim: int) -> float:
    """Multiplier folded into the Q scales: the kernel has 1/sqrt(D) built in (reference: _attention.py:130-131).
    None, a non-positive scale and NaN select the default, as the reference's op does (src/rdna4_sage/ops.py:10)."""
    if sm_scale is None or not sm_scale > 0 or math.isclose(sm_scale, head_dim ** -0.5, rel_tol=1e-6):
        return 1.0
    return float(sm_scale * math.sqrt(head_dim))


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _shape(q, k, layout):
    if layout == "HND":
        return q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3]
    return q.shape[0], q.shape[2], k.shape[2], q.shape[1], k.shape[1], q.shape[3]


def mask_view(attn_mask, q, k, layout):
    """An attn_mask with torch SDPA's semantics (bool: True = attend; a float mask of q's dtype: added to the scaled
    scores, -inf = masked; broadcastable to [B, H, q_len, kv_len]) as the kernel reads it: the mask expanded to
    [B, H, q_len, kv_len] with the key axis contiguous and broadcast axes at stride 0, its dtype code and its
    (batch, head, row) element strides.  Only the key axis is ever materialised.  Raises Unsupported for other
    dtypes and for masks that do not broadcast."""
    if not isinstance(attn_mask, torch.Tensor):
        raise Unsupported("attn_mask must be a tensor")
    if attn_mask.dtype == torch.bool:
        code = _capi.DTYPE_BOOL
    elif attn_mask.dtype == q.dtype and attn_mask.dtype in DTYPES:
        code = DTYPES[attn_mask.dtype]
    else:
        raise Unsupported(f"attn_mask dtype {attn_mask.dtype} (bool, or q's dtype {q.dtype} for an additive mask)")
    if attn_mask.device != q.device:
        raise Unsupported("attn_mask must be on the device of q")
    if attn_mask.dim() > 4:
        raise Unsupported(f"attn_mask with {attn_mask.dim()} dims")
    B, H, _, Sq, Skv, _ = _shape(q, k, layout)
    try:
        m = attn_mask.expand(B, H, Sq, Skv)
    except RuntimeError as e:
        raise Unsupported(f"attn_mask of shape {tuple(attn_mask.shape)} does not broadcast to {(B, H, Sq, Skv)}") from e
    if Skv > 1 and m.stride(3) != 1:
        base = attn_mask.reshape((1,) * (4 - attn_mask.dim()) + tuple(attn_mask.shape))
        m = base.expand(*base.shape[:3], Skv).contiguous().expand(B, H, Sq, Skv)
    return m, code, (m.stride(0), m.stride(1), m.stride(2))


def attention(q, k, v, layout="HND", sm_scale=None, is_causal=False, attn_mask=None):
    """Attention, optionally causal (bottom-right aligned, q_len <= kv_len) and / or with an attn_mask as torch SDPA
    takes it (bool: True = attend; float of q's dtype: added to the scaled scores; broadcastable to
    [B, H, q_len, kv_len]; combined with the causal mask; a query row that sees no key is 0).
    q: (B, H, Sq, D) for "HND" or (B, Sq, H, D) for "NHD"; k/v alike, with H a multiple of the kv head count.
    Returns (B, Sq, H, D) contiguous in q's dtype."""
    check_supported(q, k, v, layout, is_causal)
    if attn_mask is not None:
        mask, mcode, mstr = mask_view(attn_mask, q, k, layout)
    dev = q.device
    if layout == "HND":
        B, H, Sq, D = q.shape
        Hkv, Skv = k.shape[1], k.shape[2]
    else:
        B, Sq, H, D = q.shape
        Skv, Hkv = k.shape[1], k.shape[2]
    dt = DTYPES[q.dtype]
    q, sq_ = _bsh(q, layout)
    k, sk_ = _bsh(k, layout)
    v, sv_ = _bsh(v, layout)
    cur = torch.cuda.current_device()
    di = cur if dev.index is None else dev.index
    stream = torch._C._cuda_getCurrentRawStream(di)
    causal = bool(is_causal)
    offs, total, ws_bytes, _, _ = _forward_layout(di, B, H, Hkv, Sq, Skv, D, causal,
                                                  None if attn_mask is None else (mcode, *mstr))
    # Q8, QS, K8, KS, V8T, VS and the workspace in one caching-allocator block (torch-owned, freed with the call)
    buf = torch.empty((total,), device=dev, dtype=torch.uint8)
    base = buf.data_ptr()
    q8, qs, k8, ks, v8t, vs, ws = (base + o for o in offs)
    out = torch.empty((B, Sq, H, D), device=dev, dtype=q.dtype)
    if attn_mask is not None:
        args = ("sage_forward_masked", _ptr(q), *sq_, _ptr(k), *sk_, _ptr(v), *sv_, _ptr(out), *_out_strides(out),
                B, H, Hkv, Sq, Skv, D, dt, int(causal), qs_fold_factor(sm_scale, D), _ptr(mask), mcode, *mstr,
                q8, qs, k8, ks, v8t, vs, ws, ws_bytes, stream)
    else:
        args = ("sage_forward", _ptr(q), *sq_, _ptr(k), *sk_, _ptr(v), *sv_, _ptr(out), *_out_strides(out),
                B, H, Hkv, Sq, Skv, D, dt, int(causal), qs_fold_factor(sm_scale, D),
                q8, qs, k8, ks, v8t, vs, ws, ws_bytes, stream)
    if di == cur:
        _capi.call(*args)
    else:
        with torch.cuda.device(dev):
            _capi.call(*args)
    return out


_ALIGN = 256  # every intermediate and the workspace start on a 256-byte boundary (the library needs 16 / 256)


@functools.lru_cache(maxsize=4096)
def _forward_layout(di: int, B: int, H: int, Hkv: int, Sq: int, Skv: int, D: int, causal: bool, mask_key=None):
    """Byte offsets of Q8, QS, K8, KS, V8T, VS and the workspace inside one device buffer, the buffer's size, the
    workspace's size and the layout width (128 for head_dim 96): one caching-allocator request per call instead of
    seven.  mask_key = (mask dtype code, batch / head / row strides) for sage_forward_masked's workspace."""
    skp = _capi.kv_pad(Skv)
    dl = _capi.layout_dim(D)    # head_dim 96 is stored zero-padded to 128 channels
    if mask_key is None:
        ws_bytes = _capi.forward_workspace(di, B, H, Hkv, Sq, Skv, D, causal)
    else:
        ws_bytes = _capi.mask_workspace(di, B, H, Hkv, Sq, Skv, D, causal, *mask_key)
    sizes = (B * H * Sq * dl, B * H * Sq * 4, B * Hkv * skp * dl, B * Hkv * (skp // KV_BLOCK) * 4,
             B * Hkv * dl * skp, B * Hkv * dl * 4, ws_bytes)
    offs, at = [], 0
    for n in sizes:
        offs.append(at)
        at += (n + _ALIGN - 1) // _ALIGN * _ALIGN
    return tuple(offs), max(at, _ALIGN), ws_bytes, skp, dl


def _out_strides(out: torch.Tensor):
    # out is (B, Sq, H, D): (batch, seq, head) element strides
    return out.stride()[:3]


def lse(q, k, layout="HND", sm_scale=None, is_causal=False):
    """Row logsumexp of Q K^T * scale (natural log) over the keys, fp32 [B, H, q_len], from the 16-bit inputs on the
    gfx950 LSE kernel (the value `return_lse` returns; reference: src/sageattention/core.py:23-44).  Causal masks are
    bottom-right aligned and need q_len <= kv_len.  Raises Unsupported when the kernel cannot run these inputs."""
    if layout not in ("HND", "NHD"):
        raise Unsupported(f"layout {layout!r}")
    if not (q.is_cuda and k.device == q.device):
        raise Unsupported("tensors must be on one ROCm GPU")
    if q.dtype not in DTYPES or k.dtype != q.dtype or q.dim() != 4 or k.dim() != 4:
        raise Unsupported("4D fp16 / bf16 q and k of one dtype required")
    if device_arch(q.device) not in ARCHS:
        raise Unsupported("not a CDNA4 GPU")
    if layout == "HND":
        B, H, Sq, D = q.shape
        Hkv, Skv = k.shape[1], k.shape[2]
    else:
        B, Sq, H, D = q.shape
        Skv, Hkv = k.shape[1], k.shape[2]
    if D not in LSE_HEAD_DIMS or k.shape[-1] != D or k.shape[0] != B or Hkv == 0 or H % Hkv:
        raise Unsupported("head_dim / head counts")
    if q.numel() == 0 or k.numel() == 0 or max(q.numel(), k.numel()) > _I32_MAX:
        raise Unsupported("empty or too large")
    if is_causal and Sq > Skv:
        raise Unsupported("causal LSE needs q_len <= kv_len")
    if sm_scale is not None and not sm_scale > 0:
        # the reference's _lse takes an explicit scale as given (src/sageattention/core.py:31); the kernel's 0 means
        # the default 1 / sqrt(head_dim), so such scales go to the torch formula
        raise Unsupported("sm_scale <= 0")
    q, sq_ = _bsh(q, layout)
    k, sk_ = _bsh(k, layout)
    out = torch.empty((B, H, Sq), device=q.device, dtype=torch.float32)
    with torch.cuda.device(q.device):
        _capi.call("sage_lse_fwd", _ptr(q), *sq_, _ptr(k), *sk_, B, H, Hkv, Sq, Skv, D, DTYPES[q.dtype],
                   int(bool(is_causal)), float(sm_scale or 0.0), _ptr(out), torch.cuda.current_stream(q.device).cuda_stream)
    return out


def _packed(t: torch.Tensor):
    """(token, head) element strides of a packed [tokens, heads, D] tensor, made contiguous when the kernels cannot
    load it as 16-byte vectors (a new tensor: .contiguous() keeps a contiguous one on a misaligned base)."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 or t.stride(0) % 8 or t.stride(1) % 8:
        t = t.clone(memory_format=torch.contiguous_format)
    return t, (t.stride(0), t.stride(1))


def attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q=None, max_seqlen_k=None, sm_scale=None,
                     is_causal=False):
    """Packed variable-length attention in one stream-ordered pass (no host synchronisation): q [total_q, H, D],
    k / v [total_k, Hkv, D], cu_seqlens_q / cu_seqlens_k [batch + 1] token offsets (int32 or int64, any device).
    Sequence i is attention(q[cu_q[i]:cu_q[i+1]], k[cu_k[i]:cu_k[i+1]], v[...]) with its own quantization scales and
    a bottom-right causal mask when is_causal; query rows of a causal sequence longer than its keys that see no key
    are 0.  Rows outside every sequence are left unwritten (as torch.empty_like).  Returns [total_q, H, D].
    The reference loops over the sequences on the host (src/sageattention/core.py:80-88).  Invalid cu_seqlens
    (decreasing or past the totals) leave the output unwritten instead of raising, since they are not read back."""
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise Unsupported("tensors must be on one ROCm GPU")
    if q.dtype not in DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise Unsupported(f"dtype {q.dtype}/{k.dtype}/{v.dtype} (fp16 or bf16 required)")
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3 or k.shape != v.shape:
        raise Unsupported("packed 3D q [total_q, H, D] and k / v [total_k, Hkv, D] of one shape required")
    if device_arch(q.device) not in ARCHS:
        raise Unsupported("not a CDNA4 GPU")
    TQ, H, D = q.shape
    TK, Hkv = k.shape[0], k.shape[1]
    if D not in HEAD_DIMS or k.shape[-1] != D or Hkv == 0 or H % Hkv:
        raise Unsupported(f"head_dim {D} / heads {H} / kv heads {Hkv}")
    if cu_seqlens_q.dim() != 1 or cu_seqlens_q.shape != cu_seqlens_k.shape or cu_seqlens_q.numel() < 2:
        raise Unsupported("cu_seqlens_q / cu_seqlens_k must be 1-D of one length batch + 1 >= 2")
    if TQ == 0 or TK == 0 or max(q.numel(), k.numel()) > _I32_MAX:
        raise Unsupported("empty or too large")
    batch = cu_seqlens_q.numel() - 1
    dev = q.device
    cu_q = cu_seqlens_q.to(device=dev, dtype=torch.int32).contiguous()
    cu_k = cu_seqlens_k.to(device=dev, dtype=torch.int32).contiguous()
    q, sq_ = _packed(q)
    k, sk_ = _packed(k)
    v, sv_ = _packed(v)
    offs, total, ws_bytes = _varlen_layout(batch, H, Hkv, TQ, TK, D)
    # Q8 [H][TQ], QS, K8 / KS / V8T in the padded packed layout, VS [batch][Hkv] and the table workspace: one block
    buf = torch.empty((total,), device=dev, dtype=torch.uint8)
    q8, qs, k8, ks, v8t, vs, ws = (buf.data_ptr() + o for o in offs)
    out = torch.empty((TQ, H, D), device=dev, dtype=q.dtype)
    with torch.cuda.device(dev):
        _capi.call("sage_forward_varlen", _ptr(q), *sq_, _ptr(k), *sk_, _ptr(v), *sv_, _ptr(out), out.stride(0),
                   out.stride(1), _ptr(cu_q), _ptr(cu_k), batch, H, Hkv, TQ, TK, D, DTYPES[q.dtype],
                   int(bool(is_causal)), qs_fold_factor(sm_scale, D), q8, qs, k8, ks, v8t, vs, ws, ws_bytes,
                   torch.cuda.current_stream(dev).cuda_stream)
    return out


@functools.lru_cache(maxsize=4096)
def _varlen_layout(batch: int, H: int, Hkv: int, TQ: int, TK: int, D: int):
    """Byte offsets of the varlen pass's Q8, QS, K8, KS, V8T, VS and table workspace inside one device buffer, the
    buffer's size and the workspace's size (host arithmetic of the library's sage_varlen_layout)."""
    tkp, ws_bytes = _capi.varlen_layout(batch, H, Hkv, TQ, TK)
    dl = _capi.layout_dim(D)
    sizes = (H * TQ * dl, H * TQ * 4, Hkv * tkp * dl, Hkv * (tkp // KV_BLOCK) * 4, Hkv * dl * tkp,
             batch * Hkv * dl * 4, ws_bytes)
    offs, at = [], 0
    for n in sizes:
        offs.append(at)
        at += (n + _ALIGN - 1) // _ALIGN * _ALIGN
    return tuple(offs), max(at, _ALIGN), ws_bytes
