"""A seeded sweep of random shapes through the kernel-forced entry against the CPU emulation of the reference's math
(32-key lazy-rescale blocks, the kernel's split plan): batch, heads and GQA ratio, odd query / key lengths (one key
tile to many, causal with q_len <= kv_len), head dims 64 / 96 / 128 / 256, bf16 / fp16, HND / NHD, an explicit
sm_scale, input scales from 0.1 to 4 and outlier channels.  Same gates as the hand-picked cases: max-abs 2e-2 against
the emulation, cosine 0.999 against float attention (where the reference math itself reaches it), and the share of
output elements bit-equal to the emulation.  SAGE_SWEEP_SEED=<int> draws other shapes (the committed run uses the
default seeds)."""
import os

import numpy as np
import pytest
import torch

import cdna4_sage
from cdna4_sage import _capi
from gpu_util import assert_near_walk, cosine, hnd_np, kv_split
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
# outputs scaled up by the inputs (outlier V channels) are held to 1% of their largest magnitude instead, where one
# bf16 / fp16 step of the output (2^-8 / 2^-11 relative) already exceeds 2e-2; for outputs of order 1 it is 2e-2
REL = 1e-2
COS = 0.999
SAME_BITS = {torch.bfloat16: 0.95, torch.float16: 0.85}


def _cases(n=40, seed=20261202):
    rng = np.random.RandomState(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([64, 96, 128, 256]))
        Hkv = int(rng.randint(1, 4))
        H = Hkv * int(rng.choice([1, 2, 4]))
        B = int(rng.randint(1, 3))
        Skv = int(rng.choice([int(rng.randint(1, 130)), int(rng.randint(130, 1100))]))
        causal = bool(rng.rand() < 0.4)
        Sq = int(rng.randint(1, min(Skv, 600) + 1)) if causal else int(rng.randint(1, 600))
        dt = torch.bfloat16 if rng.rand() < 0.6 else torch.float16
        layout = "HND" if rng.rand() < 0.6 else "NHD"
        sm = None if rng.rand() < 0.7 else float(rng.uniform(0.03, 0.2))
        scale = float(np.exp(rng.uniform(np.log(0.1), np.log(4.0))))
        outliers = bool(rng.rand() < 0.3)
        out.append((i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, sm, scale, outliers))
    return out


_SEED = int(os.environ.get("SAGE_SWEEP_SEED", "0"))
CASES = _cases(seed=20261202 + _SEED)


def _ids(c):
    i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, sm, scale, outl = c
    return (f"{i}-B{B}H{H}/{Hkv}-{Sq}x{Skv}-d{D}-{'bf16' if dt == torch.bfloat16 else 'f16'}-{layout}"
            f"{'-causal' if causal else ''}{'-sm' if sm else ''}{'-outl' if outl else ''}")


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_random_shapes_vs_emulation(dev, case):
    i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, sm, scale, outliers = case
    g = torch.Generator().manual_seed(1000 + i)
    q = torch.randn(B, H, Sq, D, generator=g) * scale
    k = torch.randn(B, Hkv, Skv, D, generator=g) * scale
    v = torch.randn(B, Hkv, Skv, D, generator=g)
    if outliers:  # a few channels x10, as in activations with massive channels
        ch = torch.randperm(D, generator=g)[:3]
        q[..., ch] *= 10
        k[..., ch] *= 10
        v[..., ch[:1]] *= 10
    q, k, v = (t.to(dt) for t in (q, k, v))
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), tensor_layout=layout, sm_scale=sm, is_causal=causal)
    assert out.shape == q.shape and out.dtype == dt
    got = hnd_np(out, layout)
    qn, kn, vn = hnd_np(q, layout), hnd_np(k, layout), hnd_np(v, layout)
    q8, qs = orc.quant_q(qn, sm)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(Skv))
    split = kv_split(dev, B, H, Sq, Skv, D, causal)
    emu = orc.attention(q8, qs, k8, ks, v8, vs, Skv, causal=causal, block_n=32,
                        out_dtype="bf16" if dt == torch.bfloat16 else "f16", kv_split=split,
                        also_unsplit=split is not None)
    emu, walk = emu if split is not None else (emu, None)
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal, sm_scale=sm)
    err = float(np.abs(got - emu).max())
    assert err <= max(MAX_ABS, REL * float(np.abs(emu).max())), (err, float(np.abs(emu).max()))
    assert cosine(got, ref) >= min(COS, cosine(emu, ref) - 1e-4)
    assert float((got == emu).mean()) >= SAME_BITS[dt]
    if walk is not None:   # split tiles, also against the reference's one walk over every key
        assert_near_walk(got, walk, ref)


def _mask_cases(n=20, seed=777):
    rng = np.random.RandomState(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([64, 96, 128, 256]))
        Hkv = int(rng.randint(1, 3))
        H = Hkv * int(rng.choice([1, 2]))
        B = int(rng.randint(1, 3))
        Skv = int(rng.randint(1, 900))
        causal = bool(rng.rand() < 0.3)
        Sq = int(rng.randint(1, min(Skv, 400) + 1)) if causal else int(rng.randint(1, 400))
        dt = torch.bfloat16 if rng.rand() < 0.6 else torch.float16
        layout = "HND" if rng.rand() < 0.6 else "NHD"
        shape = [(Skv,), (1, 1, 1, Skv), (B, 1, 1, Skv), (Sq, Skv), (1, H, Sq, Skv), (B, H, Sq, Skv)][rng.randint(6)]
        kind = ["bool", "bool", "bool", "float"][rng.randint(4)]
        p = float(rng.choice([0.3, 0.7, 0.95, 1.0]))
        out.append((i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, shape, kind, p))
    return out


MASK_CASES = _mask_cases(seed=777 + _SEED)


def _mask_ids(c):
    i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, shape, kind, p = c
    return (f"{i}-B{B}H{H}/{Hkv}-{Sq}x{Skv}-d{D}-{'bf16' if dt == torch.bfloat16 else 'f16'}-{layout}"
            f"{'-causal' if causal else ''}-{kind}{list(shape)}-p{p}")


@pytest.mark.parametrize("case", MASK_CASES, ids=[_mask_ids(c) for c in MASK_CASES])
def test_random_masks_vs_emulation(dev, case):
    """Random bool masks (density 0.3 to 1, any broadcast shape torch SDPA takes) and additive masks of the inputs'
    dtype (0 where a bool mask is True, -inf elsewhere, plus a bias of up to +-4 on the visible keys)."""
    i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, shape, kind, p = case
    g = torch.Generator().manual_seed(5000 + i)
    q = torch.randn(B, H, Sq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    keep = torch.rand(shape, generator=g) < p
    if kind == "bool":
        mask = keep
    else:
        bias = (torch.rand(shape, generator=g) * 8 - 4)
        mask = torch.where(keep, bias, torch.full_like(bias, float("-inf"))).to(dt)
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), tensor_layout=layout, is_causal=causal,
                               attn_mask=mask.to(dev))
    assert out.shape == q.shape and out.dtype == dt
    got = hnd_np(out, layout)
    assert np.isfinite(got).all()
    qn, kn, vn = hnd_np(q, layout), hnd_np(k, layout), hnd_np(v, layout)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(Skv))
    m = torch.broadcast_to(mask, (B, H, Sq, Skv))
    m = m.numpy() if kind == "bool" else m.float().numpy()
    split = kv_split(dev, B, H, Sq, Skv, D, False)
    emu = orc.attention(q8, qs, k8, ks, v8, vs, Skv, causal=causal, block_n=32,
                        out_dtype="bf16" if dt == torch.bfloat16 else "f16", kv_split=split, attn_mask=m,
                        also_unsplit=split is not None)
    emu, walk = emu if split is not None else (emu, None)
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal, attn_mask=m)
    err = float(np.abs(got - emu).max())
    assert err <= max(MAX_ABS, REL * float(np.abs(emu).max())), (err, float(np.abs(emu).max()))
    assert cosine(got, ref) >= min(COS, cosine(emu, ref) - 1e-4)
    assert float((got == emu).mean()) >= SAME_BITS[dt]
    if walk is not None:
        assert_near_walk(got, walk, ref)
