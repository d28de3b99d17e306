"""gfx950 attention kernel vs the CPU emulation of the reference's quantized math and vs float attention.

Tolerances (north star): max |out - emulation| <= 2e-2 with the emulation run at the kernel's own 64-key tile, and
cosine >= 0.999 against float attention; the reference's own gate is cosine > 0.998 (tests/test_attention.py:175).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cdna4_sage
from cdna4_sage import _capi
from gpu_util import cosine, hnd_np
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
COS = 0.999

CASES = [  # B, H, Hkv, Sq, Skv, D, dtype, layout, causal
    (1, 2, 2, 300, 300, 128, torch.bfloat16, "HND", False),
    (2, 4, 2, 515, 515, 64, torch.float16, "NHD", False),
    (1, 2, 2, 1000, 1000, 128, torch.bfloat16, "HND", True),
    (1, 4, 1, 257, 257, 64, torch.bfloat16, "HND", True),
    (1, 2, 2, 130, 777, 128, torch.float16, "HND", False),
    (1, 3, 3, 1024, 64, 128, torch.bfloat16, "NHD", False),
    (3, 2, 2, 77, 1031, 128, torch.bfloat16, "HND", False),
    (1, 8, 8, 1024, 1024, 64, torch.bfloat16, "HND", False),   # config 1 shape
]


def _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    return q, k, v


def _emulate(q, k, v, layout, causal, sm_scale=None, out_dtype="bf16"):
    qn, kn, vn = hnd_np(q, layout), hnd_np(k, layout), hnd_np(v, layout)
    q8, qs = orc.quant_q(qn, sm_scale)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(kn.shape[2]))
    emu = orc.attention(q8, qs, k8, ks, v8, vs, kn.shape[2], causal=causal, block_n=64, out_dtype=out_dtype)
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal, sm_scale=sm_scale)
    return emu, ref


@pytest.mark.parametrize("B,H,Hkv,Sq,Skv,D,dt,layout,causal", CASES)
def test_attention_vs_emulation(dev, B, H, Hkv, Sq, Skv, D, dt, layout, causal):
    q, k, v = _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=Sq + Skv)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), tensor_layout=layout, is_causal=causal)
    assert out.shape == q.shape and out.dtype == dt
    got = hnd_np(out, layout)
    emu, ref = _emulate(q, k, v, layout, causal, out_dtype="bf16" if dt == torch.bfloat16 else "f16")
    err = float(np.abs(got - emu).max())
    c = cosine(got, ref)
    assert err <= MAX_ABS, err
    assert c >= COS, c


def test_sm_scale(dev):
    q, k, v = _inputs(1, 2, 2, 600, 600, 128, torch.bfloat16, "HND", seed=7)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND", sm_scale=0.05)
    emu, ref = _emulate(q, k, v, "HND", False, sm_scale=0.05)
    got = hnd_np(out)
    assert float(np.abs(got - emu).max()) <= MAX_ABS
    assert cosine(got, ref) >= COS


def test_flux_config2_full(dev):
    """Config 2 (Flux 1x24x4608x128 bf16, outlier K channels): cosine vs fp32 attention on all heads, and the
    emulation on a two-head sample (the per-head computation is independent of the other heads)."""
    from cdna4_sage.configs import CONFIGS, make_inputs

    cfg = CONFIGS["2"]
    q, k, v = make_inputs(cfg)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND")
    ref = F.scaled_dot_product_attention(q.to(dev).float(), k.to(dev).float(), v.to(dev).float())
    c = F.cosine_similarity(out.float().flatten(), ref.flatten(), dim=0).item()
    assert c >= COS, c
    qs_, ks_, vs_ = make_inputs(cfg, heads=slice(5, 7))
    emu, _ = _emulate(qs_, ks_, vs_, "HND", False)
    got = out[:, 5:7].float().cpu().numpy()
    assert float(np.abs(got - emu).max()) <= MAX_ABS


@pytest.mark.parametrize("D", [96, 256])
def test_unsupported_head_dims(dev, D):
    q = torch.randn(1, 2, 256, D, device=dev, dtype=torch.bfloat16)
    with pytest.raises(cdna4_sage.Unsupported):
        cdna4_sage.attention(q, q, q, "HND")
