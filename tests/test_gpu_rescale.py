"""The reference's per-32-key lazy rescale on inputs that move a row's max inside a 64-key tile, and head dim 256 at
its extreme scores.

Staircase inputs: keys rise by more than 8 log2 units of logit every 32 keys for the even query rows (odd rows are
plain random), so every 64-key tile has rows whose max moves at its second 32-key block.  The kernel's waves then run
those tiles in two passes (block 0 alone, then block 1 with its rescale first); the emulation takes the reference's
decisions once per 32-key block (kernel_build/make_sage_r2.py:180-190).  Each case checks, on the CPU, that the
inputs really contain such block-1 rescales.

Plateau inputs: from the second 64-key tile on, the even query rows see keys about 6.5 log2 units above the first
tile's max, never the 8 that moves it.  Once a wave's rows all have a max, the kernel starts each tile with a
speculative pass (no block maxima; it stands when every lane's sum of 16 probabilities is below 2^7.5); here those
sums reach ~900, so the speculative passes do not stand, the exact passes find no row whose max moves, and the
results must still be the reference's.  The case checks, on the CPU, that such tiles occur.

Head dim 256: Q and K with one dominant channel per 128-channel rotation block, anti-aligned, quantize to
S = Q8 K8^T down to -127^2 * 256 = -4,129,024, below the range a seeded fp32 read of the int32 accumulator covers
(S >= -2,292,099); the kernel converts S exactly there.  Dense, additive-mask and varlen paths.

Tolerances: max |out - emulation| <= 2e-2 and <= 1% of max |emulation|, as for every attention gate.  Against float
attention the staircase inputs are hard on the quantization itself (K is dominated by the shared direction, so its
noise part gets few int8 levels): the emulation of the reference's math reaches cosine 0.9978-0.9994 there, so the
kernel is held to the emulation's own cosine less 1e-4; the head dim 256 cases keep cosine >= 0.999.
"""
import math

import numpy as np
import pytest
import torch

import cdna4_sage
from cdna4_sage import _capi
from gpu_util import cosine, hnd_np, kv_split
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
COS = 0.999
SEEDED_MIN_S = -2292099


def _staircase(B, H, Hkv, S, D, dt, seed, step=1.0):
    """Even query rows carry a shared direction u (|u|^2 = D); key j carries (j // 32) * step * u, so each 32-key
    block raises those rows' logits by about step * sqrt(D) * log2(e) log2 units (11.5 at D = 64)."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(D, generator=g)
    u = u / u.norm() * math.sqrt(D)
    q = torch.randn(B, H, S, D, generator=g) * 0.5
    q[:, :, 0::2] += u
    k = torch.randn(B, Hkv, S, D, generator=g) * 0.5
    k += (step * (torch.arange(S) // 32).float())[:, None] * u
    v = torch.randn(B, Hkv, S, D, generator=g)
    return q.to(dt), k.to(dt), v.to(dt)


def _block1_rescales(q8, qs, k8, ks, seq_kv, causal):
    """Count (row, 64-key tile) pairs whose max moves at the tile's second 32-key block under the reference's
    decisions (threshold 8 in log2 units)."""
    B, H, Sq, D = q8.shape
    hk = np.arange(H) // (H // k8.shape[1])
    cl = (orc.logit_scale_base(D) * qs).astype(np.float32)
    s = np.matmul(q8.astype(np.float32), np.swapaxes(k8.astype(np.float32)[:, hk], -1, -2))
    cols = np.arange(s.shape[-1])
    mask = cols[None, :] >= seq_kv
    if causal:
        mask = mask | (cols[None, :] > np.arange(Sq)[:, None] + seq_kv - Sq)
    s = np.where(mask, -np.inf, s)
    nb = s.shape[-1] // 32
    bm = s.reshape(B, H, Sq, nb, 32).max(-1) * ks[:, hk][:, :, None, :nb]
    m = np.full((B, H, Sq), -np.inf, np.float32)
    count = 0
    for b in range(nb):
        mc = np.maximum(m, bm[..., b])
        with np.errstate(invalid="ignore"):
            need = (mc - m) * cl > 8
        if b % 2 == 1:
            count += int(need.sum())
        m = np.where(need, mc, m)
    return count


STAIR_CASES = [  # B, H, Hkv, S, D, dtype, causal
    (1, 2, 2, 300, 64, torch.bfloat16, False),
    (1, 4, 2, 333, 128, torch.float16, True),
    (2, 2, 1, 260, 128, torch.bfloat16, False),
    (1, 2, 2, 200, 256, torch.bfloat16, True),
    (1, 2, 2, 300, 96, torch.bfloat16, False),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,dt,causal", STAIR_CASES)
def test_block1_rescales_follow_the_reference_decisions(dev, B, H, Hkv, S, D, dt, causal):
    q, k, v = _staircase(B, H, Hkv, S, D, dt, seed=S + D)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND", is_causal=causal)
    got = hnd_np(out)
    qn, kn, vn = hnd_np(q), hnd_np(k), hnd_np(v)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
    assert _block1_rescales(q8, qs, k8, ks, S, causal) >= 100
    od = "bf16" if dt == torch.bfloat16 else "f16"
    split = kv_split(dev, B, H, S, S, D, causal)
    emu = orc.attention(q8, qs, k8, ks, v8, vs, S, causal=causal, block_n=32, out_dtype=od, kv_split=split)
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS, err
    assert err <= 1e-2 * float(np.abs(emu).max()), err
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal)
    assert cosine(got, ref) >= min(COS, cosine(emu, ref) - 1e-4)


def test_block1_rescales_with_masks(dev):
    """The same staircase through the mask variant: a bool key-padding mask (bit-masked tiles) and an additive mask
    of small biases (the bias path, whose row max is taken over the biased logits per 32-key block)."""
    B, H, S, D = 1, 2, 300, 128
    q, k, v = _staircase(B, H, H, S, D, torch.bfloat16, seed=5)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    qn, kn, vn = hnd_np(q), hnd_np(k), hnd_np(v)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
    assert _block1_rescales(q8, qs, k8, ks, S, False) >= 100
    g = torch.Generator().manual_seed(6)
    pad = torch.arange(S)[None, None, None, :] < 270
    bias = (torch.rand(1, 1, S, S, generator=g) - 0.5).to(torch.bfloat16)
    split = kv_split(dev, B, H, S, S, D, False)
    for mask in (pad, bias):
        out = cdna4_sage.attention(qd, kd, vd, "HND", attn_mask=mask.to(dev))
        got = hnd_np(out)
        m = mask.numpy() if mask.dtype == torch.bool else mask.float().numpy()
        emu = orc.attention(q8, qs, k8, ks, v8, vs, S, block_n=32, out_dtype="bf16", kv_split=split, attn_mask=m)
        assert float(np.abs(got - emu).max()) <= MAX_ABS
        ref = orc.sdpa_reference(qn, kn, vn, attn_mask=m)
        assert cosine(got, ref) >= min(COS, cosine(emu, ref) - 1e-4)



def _plateau(B, H, Hkv, S, D, dt, seed, rise=6.5):
    """Even query rows carry a shared direction u (|u|^2 = D) plus small noise; keys from 64 on carry c * u with
    c * sqrt(D) * log2(e) = rise, so those rows' logits sit `rise` log2 units above the first tile's."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(D, generator=g)
    u = u / u.norm() * math.sqrt(D)
    q = torch.randn(B, H, S, D, generator=g) * 0.2
    q[:, :, 0::2] += u
    k = torch.randn(B, Hkv, S, D, generator=g) * 0.2
    k[:, :, 64:] += rise / (math.sqrt(D) * math.log2(math.e)) * u
    v = torch.randn(B, Hkv, S, D, generator=g)
    return q.to(dt), k.to(dt), v.to(dt)


def _speculative_false_alarms(q8, qs, k8, ks, seq_kv, causal):
    """(wave of 32 query rows, 64-key tile) pairs in which every row has a max before the tile, some lane's sum of
    its 16 probabilities of a 32-key block (keys 32 kb + 4 hf + 8 g + r, g, r < 4) reaches 181, and the reference's
    decisions move no row's max: the speculative passes that must give way to an exact pass that changes nothing."""
    B, H, Sq, D = q8.shape
    hk = np.arange(H) // (H // k8.shape[1])
    cl = (orc.logit_scale_base(D) * qs).astype(np.float32)
    s = np.matmul(q8.astype(np.float32), np.swapaxes(k8.astype(np.float32)[:, hk], -1, -2))
    cols = np.arange(s.shape[-1])
    mask = cols[None, :] >= seq_kv
    if causal:
        mask = mask | (cols[None, :] > np.arange(Sq)[:, None] + seq_kv - Sq)
    s = np.where(mask, -np.inf, s)
    ksx = np.repeat(ks[:, hk], 32, axis=-1)[..., :s.shape[-1]]
    lane = [np.array([32 * kb + 4 * hf + 8 * g + r for g in range(4) for r in range(4)]) for kb in (0, 1)
            for hf in (0, 1)]
    m = np.full((B, H, Sq), -np.inf, np.float32)
    count = 0
    for t in range(s.shape[-1] // 64):
        blk = s[..., 64 * t: 64 * t + 64] * ksx[..., None, 64 * t: 64 * t + 64]
        m_prev = m.copy()
        moved = np.zeros_like(m, dtype=bool)
        for kb in (0, 1):
            mc = np.maximum(m, blk[..., 32 * kb: 32 * kb + 32].max(-1))
            with np.errstate(invalid="ignore"):
                need = (mc - m) * cl > 8
            moved |= need
            m = np.where(need, mc, m)
        with np.errstate(invalid="ignore", over="ignore"):
            p = np.exp2((blk - m_prev[..., None]) * cl[..., None])
        big = np.zeros_like(moved)
        for keys in lane:
            big |= p[..., keys].sum(-1) >= 181.0
        for w in range(0, Sq, 32):
            rows = slice(w, min(w + 32, Sq))
            finite = np.isfinite(m_prev[..., rows]).all(-1)
            count += int((finite & big[..., rows].any(-1) & ~moved[..., rows].any(-1)).sum())
    return count


@pytest.mark.parametrize("D,dt,causal", [(128, torch.bfloat16, False), (64, torch.float16, True)])
def test_speculative_passes_that_do_not_stand(dev, D, dt, causal):
    B, H, S = 1, 2, 400
    q, k, v = _plateau(B, H, H, S, D, dt, seed=7 + D)
    qn, kn, vn = hnd_np(q), hnd_np(k), hnd_np(v)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
    assert _speculative_false_alarms(q8, qs, k8, ks, S, causal) >= 20
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND", is_causal=causal)
    got = hnd_np(out)
    split = kv_split(dev, B, H, S, S, D, causal)
    emu = orc.attention(q8, qs, k8, ks, v8, vs, S, causal=causal, block_n=32, out_dtype="bf16" if dt == torch.bfloat16
                        else "f16", kv_split=split)
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS and err <= 1e-2 * float(np.abs(emu).max()), err
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal)
    assert cosine(got, ref) >= min(COS, cosine(emu, ref) - 1e-4)

def _anti_aligned_d256(B, H, Hkv, Sq, Skv, dt, seed):
    """Q rows with one dominant channel in each 128-channel block; K rows with the same channels negated and scaled
    by a_j in [4, 8]: after the block Hadamard every element of a block is +-8 (Q) and -+a_j (K), so S_j runs from
    -4,129,024 (a_j = 8) to about half of it."""
    g = torch.Generator().manual_seed(seed)
    c1, c2 = 5, 128 + 77
    q = torch.randn(B, H, Sq, 256, generator=g) * 0.002
    q[..., c1] += 8.0
    q[..., c2] += 8.0
    k = torch.randn(B, Hkv, Skv, 256, generator=g) * 0.002
    a = 4.0 + 4.0 * torch.rand(B, Hkv, Skv, generator=g)
    a[..., ::7] = 8.0
    k[..., c1] -= a
    k[..., c2] -= a
    v = torch.randn(B, Hkv, Skv, 256, generator=g)
    return q.to(dt), k.to(dt), v.to(dt)


def _min_s(q8, k8):
    hk = np.arange(q8.shape[1]) // (q8.shape[1] // k8.shape[1])
    return float(np.matmul(q8.astype(np.float64), np.swapaxes(k8.astype(np.float64)[:, hk], -1, -2)).min())


@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_256_extreme_scores_dense_and_masked(dev, causal):
    B, H, Hkv, S = 1, 4, 2, 300
    q, k, v = _anti_aligned_d256(B, H, Hkv, S, S, torch.bfloat16, seed=21 + causal)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    qn, kn, vn = hnd_np(q), hnd_np(k), hnd_np(v)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
    assert _min_s(q8, k8) < 1.6 * SEEDED_MIN_S
    split = kv_split(dev, B, H, S, S, 256, causal)
    out = cdna4_sage.attention(qd, kd, vd, "HND", is_causal=causal)
    got = hnd_np(out)
    emu = orc.attention(q8, qs, k8, ks, v8, vs, S, causal=causal, block_n=32, kv_split=split)
    assert float(np.abs(got - emu).max()) <= MAX_ABS
    assert cosine(got, orc.sdpa_reference(qn, kn, vn, causal=causal)) >= COS
    # additive mask (the bias path reads the same scores)
    g = torch.Generator().manual_seed(30)
    bias = ((torch.rand(1, 1, S, S, generator=g) - 0.5) * 2.0).to(torch.bfloat16)
    out = cdna4_sage.attention(qd, kd, vd, "HND", is_causal=causal, attn_mask=bias.to(dev))
    got = hnd_np(out)
    m = bias.float().numpy()
    emu = orc.attention(q8, qs, k8, ks, v8, vs, S, causal=causal, block_n=32, kv_split=split, attn_mask=m)
    assert float(np.abs(got - emu).max()) <= MAX_ABS
    assert cosine(got, orc.sdpa_reference(qn, kn, vn, causal=causal, attn_mask=m)) >= COS


def test_head_dim_256_extreme_scores_varlen(dev):
    lq, lk = [200, 333], [260, 500]
    H, Hkv = 4, 2
    qs_, ks_, vs_ = [], [], []
    for i, (a, b) in enumerate(zip(lq, lk)):
        q, k, v = _anti_aligned_d256(1, H, Hkv, a, b, torch.float16, seed=40 + i)
        qs_.append(q[0].transpose(0, 1))
        ks_.append(k[0].transpose(0, 1))
        vs_.append(v[0].transpose(0, 1))
    q, k, v = (torch.cat(t).contiguous() for t in (qs_, ks_, vs_))          # [total, heads, 256]
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q8, _ = orc.quant_q(hnd_np(q[None], "NHD"))
    k8, *_ = orc.quant_kv(hnd_np(k[None], "NHD")[:, :, :lk[0]], hnd_np(v[None], "NHD")[:, :, :lk[0]])
    assert _min_s(q8[:, :, :lq[0]], k8) < 1.6 * SEEDED_MIN_S
    out = cdna4_sage.attention_varlen(q.to(dev), k.to(dev), v.to(dev), torch.tensor(cu_q, device=dev),
                                      torch.tensor(cu_k, device=dev), max(lq), max(lk))
    emu = orc.sage_forward_varlen(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                  block_n=32, out_dtype="f16")
    got = out.float().cpu().numpy()
    assert float(np.abs(got - emu).max()) <= MAX_ABS
    for i in range(2):
        q0, q1, k0, k1 = cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]
        hnd = lambda t: np.ascontiguousarray(t.float().numpy().transpose(1, 0, 2))[None]   # noqa: E731
        ref = orc.sdpa_reference(hnd(q[q0:q1]), hnd(k[k0:k1]), hnd(v[k0:k1]))[0].transpose(1, 0, 2)
        assert cosine(got[q0:q1], ref) >= COS


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_staircase_and_plateau(dev, causal):
    """The packed variable-length kernel runs the same tile passes: a staircase sequence (block-1 rescales after
    the first tile) and a plateau sequence (speculative passes that do not stand) in one batch."""
    H, Hkv, D = 4, 2, 128
    lq, lk = [300, 260], [300, 400]
    gens = [lambda a, b: _staircase(1, H, Hkv, max(a, b), D, torch.bfloat16, seed=70 + causal),
            lambda a, b: _plateau(1, H, Hkv, max(a, b), D, torch.bfloat16, seed=80 + causal)]
    qs_, ks_, vs_ = [], [], []
    for g, a, b in zip(gens, lq, lk):
        q, k, v = g(a, b)
        qs_.append(q[0, :, :a].transpose(0, 1))
        ks_.append(k[0, :, :b].transpose(0, 1))
        vs_.append(v[0, :, :b].transpose(0, 1))
    q, k, v = (torch.cat(t).contiguous() for t in (qs_, ks_, vs_))          # [total, heads, D]
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    # the inputs do contain both kinds of tile (counted per sequence on the CPU)
    hnd = lambda t: np.ascontiguousarray(t.float().numpy().transpose(1, 0, 2))[None]   # noqa: E731
    q8a, qsa = orc.quant_q(hnd(q[:lq[0]]))
    k8a, ksa, _, _ = orc.quant_kv(hnd(k[:lk[0]]), hnd(v[:lk[0]]), seq_pad=_capi.kv_pad(lk[0]))
    assert _block1_rescales(q8a, qsa, k8a, ksa, lk[0], causal) >= 50
    q8b, qsb = orc.quant_q(hnd(q[lq[0]:]))
    k8b, ksb, _, _ = orc.quant_kv(hnd(k[lk[0]:]), hnd(v[lk[0]:]), seq_pad=_capi.kv_pad(lk[1]))
    assert _speculative_false_alarms(q8b, qsb, k8b, ksb, lk[1], causal) >= 10
    out = cdna4_sage.attention_varlen(q.to(dev), k.to(dev), v.to(dev), torch.tensor(cu_q, device=dev),
                                      torch.tensor(cu_k, device=dev), max(lq), max(lk), is_causal=causal)
    emu = orc.sage_forward_varlen(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                  causal=causal, block_n=32, out_dtype="bf16")
    got = out.float().cpu().numpy()
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS and err <= 1e-2 * float(np.abs(emu).max()), err


@pytest.mark.parametrize("scale,D,causal", [(30.0, 128, False), (300.0, 128, True), (1000.0, 64, False)])
def test_large_logits(dev, scale, D, causal):
    """Inputs scaled so that the logits reach ~10^3-10^6 log2 units: the speculative pass's exponent arguments and
    the reference's rescale test then differ by more fp32 rounding, the softmax is close to one-hot, and the output
    must still follow the emulation within the usual bounds."""
    B, H, S = 1, 2, 333
    g = torch.Generator().manual_seed(int(scale) + D)
    q = (torch.randn(B, H, S, D, generator=g) * scale).to(torch.bfloat16)
    k = (torch.randn(B, H, S, D, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND", is_causal=causal)
    got = hnd_np(out)
    qn, kn, vn = hnd_np(q), hnd_np(k), hnd_np(v)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
    assert np.isfinite(got).all()
    split = kv_split(dev, B, H, S, S, D, causal)
    emu = orc.attention(q8, qs, k8, ks, v8, vs, S, causal=causal, block_n=32, kv_split=split)
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS and err <= 1e-2 * float(np.abs(emu).max()), err


@pytest.mark.parametrize("kind", ["bool", "bias", "varlen"])
def test_large_logits_mask_and_varlen(dev, kind):
    """The large-scale read (scores taken exactly, the reference's offset) in the mask variant's bit-masked and
    additive-bias bodies and in the packed variable-length kernel."""
    H, D, scale = 2, 128, 300.0
    g = torch.Generator().manual_seed(91)
    if kind == "varlen":
        lq, lk = [150, 260], [200, 260]
        q = (torch.randn(sum(lq), H, D, generator=g) * scale).to(torch.bfloat16)
        k = (torch.randn(sum(lk), H, D, generator=g) * scale).to(torch.bfloat16)
        v = torch.randn(sum(lk), H, D, generator=g).to(torch.bfloat16)
        cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
        cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
        out = cdna4_sage.attention_varlen(q.to(dev), k.to(dev), v.to(dev), torch.tensor(cu_q, device=dev),
                                          torch.tensor(cu_k, device=dev), max(lq), max(lk))
        got = out.float().cpu().numpy()
        emu = orc.sage_forward_varlen(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                      block_n=32, out_dtype="bf16")
    else:
        B, S = 1, 300
        q = (torch.randn(B, H, S, D, generator=g) * scale).to(torch.bfloat16)
        k = (torch.randn(B, H, S, D, generator=g) * scale).to(torch.bfloat16)
        v = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
        if kind == "bool":
            mask = torch.rand(1, 1, S, S, generator=g) < 0.6
            mask[..., 0] = True
            m = mask.numpy()
        else:
            mask = ((torch.rand(1, 1, S, S, generator=g) - 0.5) * 8).to(torch.bfloat16)
            m = mask.float().numpy()
        out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND", attn_mask=mask.to(dev))
        got = hnd_np(out)
        qn, kn, vn = hnd_np(q), hnd_np(k), hnd_np(v)
        q8, qs = orc.quant_q(qn)
        k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
        cl = (orc.logit_scale_base(D) * qs).astype(np.float32)
        assert orc.wide_rows(cl, ks, S, np.arange(S), np.arange(H)).all()
        split = kv_split(dev, B, H, S, S, D, False)
        emu = orc.attention(q8, qs, k8, ks, v8, vs, S, block_n=32, kv_split=split, attn_mask=m)
    assert np.isfinite(got).all()
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS and err <= 1e-2 * float(np.abs(emu).max()), err
