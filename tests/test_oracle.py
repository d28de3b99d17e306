"""Pins the CPU oracle (oracle/sage_oracle.py) with checks that do not restate its formulas: closed forms, exact
rational arithmetic, torch's own E4M3 cast and inf-norm (the ops the reference calls), invariants of the quantizers
and brute-force attention on cases whose answer is known."""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import sage_oracle as orc

F32 = np.float32


def rn32(x: Fraction) -> np.float32:
    """Correctly rounded float32 (round to nearest even) of an exact rational."""
    if x == 0:
        return F32(0.0)
    s = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    qn = a / ulp
    n = qn.numerator // qn.denominator
    rem = qn - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return F32(s * float(n * ulp))


# ------------------------------------------------------------------------------------------------ Hadamard
@pytest.mark.parametrize("d", [1, 2, 4, 64, 128])
def test_hadamard_closed_form(d):
    h = orc.hadamard_pm1(d)
    i = np.arange(d)
    popc = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    assert np.array_equal(h, (-1.0) ** popc)                      # H[i, j] = (-1)^popcount(i & j)
    assert np.array_equal(h @ h.T, d * np.eye(d))                  # H H^T = d I


@pytest.mark.parametrize("d", [64, 128])
def test_fwht_matches_matrix_and_special_cases(d):
    h = orc.hadamard_pm1(d)
    eye = np.eye(d)
    assert np.array_equal(orc.fwht_rows(eye), h)                    # e_i -> row i of H
    c = np.full((3, d), 0.375)
    exp = np.zeros((3, d))
    exp[:, 0] = d * 0.375
    assert np.array_equal(orc.fwht_rows(c), exp)                     # constant row -> d * c * e_0
    x = np.random.default_rng(0).integers(-1000, 1000, (5, d)).astype(np.float64)
    assert np.array_equal(orc.fwht_rows(x), x @ h)                  # exact on integers


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fwht_float32_is_correctly_rounded_exact_sum(dtype):
    """The rotation used by the kernels is RN32 of the exact +-1 sum (checked with rational arithmetic)."""
    d = 128
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(6, d, generator=g) * torch.exp2(torch.randint(-8, 8, (6, d), generator=g).float())).to(dtype)
    xs = x.float().numpy()
    got = orc.fwht_rows(xs).astype(F32)
    h = orc.hadamard_pm1(d).astype(int)
    for r in range(xs.shape[0]):
        fr = [Fraction(float(v)) for v in xs[r]]
        for j in range(0, d, 7):
            exact = sum((fr[i] if h[i, j] > 0 else -fr[i]) for i in range(d))
            assert got[r, j] == rn32(exact), (r, j)


# ------------------------------------------------------------------------------------------------ rounding helpers
def test_round_half_away_matches_exact_definition():
    """int8 conversion = trunc(RN32(y +- 0.5)) (reference: sage_quant.py:44): ties go away from zero and values
    just below a half can still round up through the fp32 addition."""
    ys = [0.5, -0.5, 1.5, -1.5, 2.5, 126.5, -126.5, 0.49999997, -0.49999997, 0.0, -0.0, 127.0, -127.0, 3.4999998]
    ys += list(np.random.default_rng(2).uniform(-127.4, 127.4, 2000).astype(F32))
    got = orc.round_half_away_i8(np.array(ys, dtype=F32))
    for y, q in zip(ys, got):
        y = F32(y)
        t = rn32(Fraction(float(y)) + (Fraction(1, 2) if y >= 0 else Fraction(-1, 2)))
        assert int(q) == int(math.trunc(float(t))), y
    assert orc.round_half_away_i8(np.array([0.5 - 2**-25], dtype=F32))[0] == 1   # fp32(y + 0.5) == 1.0


def _all_finite_e4m3():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    return codes, torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()


def test_e4m3_decode_matches_torch():
    codes, vals = _all_finite_e4m3()
    assert np.array_equal(orc.e4m3_to_f32(codes), vals)


def test_e4m3_encode_matches_torch_cast():
    """fp32 -> E4M3FN (RNE with subnormals) against torch's own cast, exhaustively on every code, every midpoint
    between neighbouring codes (ties to even) and their fp32 neighbours, plus random values in [-448, 448]."""
    codes, vals = _all_finite_e4m3()
    pos = np.unique(vals[vals >= 0])
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(F32)
    cand = np.concatenate([pos, mids, np.nextafter(mids, F32(0)), np.nextafter(mids, F32(1000))])
    cand = np.concatenate([cand, -cand, np.random.default_rng(3).uniform(-448, 448, 200000).astype(F32),
                           (np.random.default_rng(4).standard_normal(20000) * 2.0 ** -8).astype(F32)])
    cand = np.clip(cand, F32(-448), F32(448)).astype(F32)
    ref = torch.from_numpy(cand).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.f32_to_e4m3(cand), ref)


def test_division_sequence_of_the_kernels():
    """The HIP quantizers divide by a shared scale s as y0 = x*r, e = fma(-y0, s, x), y = fma(e, r, y0) with
    r = RN(1/s).  Exact rational arithmetic shows this equals IEEE RN(x / s), including adversarial scales whose
    significand is all ones and quotients next to rounding ties."""
    rng = np.random.default_rng(5)
    cases = []
    for _ in range(3000):
        a = max(F32(abs(rng.standard_normal()) * 10 ** rng.uniform(-6, 3)), F32(1e-12))
        s = F32(a / F32(127.0))
        cases.append((F32(rng.uniform(-1, 1) * a), s))
    for kk in range(500):
        s = np.frombuffer(struct.pack("<I", 0x3F7FFFFF - kk), dtype=F32)[0] * F32(2.0 ** rng.integers(-20, 5))
        x = F32(F32(rng.integers(-127, 128) + 0.5) * s)
        cases += [(x, s), (np.nextafter(x, F32(np.inf)), s)]
    fma = lambda a, b, c: rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))  # noqa: E731
    for x, s in cases:
        r = rn32(Fraction(1) / Fraction(float(s)))
        y0 = F32(x * r)
        y = fma(fma(-y0, s, x), r, y0)
        assert y == F32(x / s), (x, s)


# ------------------------------------------------------------------------------------------------ quantizers
def _bf16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16).float().numpy()


def test_quant_q_invariants():
    q = _bf16((2, 3, 97, 128), 6)
    q[0, 0, 4] = 0.0
    q8, qs = orc.quant_q(q)
    x = orc.fwht_rows(q).astype(F32)
    amax = np.abs(x).max(-1)
    nz = amax > 1e-12
    assert np.all(np.abs(q8.astype(int)).max(-1)[nz] == 127)         # full int8 range on every row
    s = qs * 128                                                      # QS = s / RB, RB = head_dim
    assert np.allclose(s[nz] * 127, amax[nz], rtol=1e-6)
    assert np.all(np.abs(q8 * s[..., None] - x) <= s[..., None] * 0.5 * (1 + 1e-5))   # |dequant error| <= s/2
    assert np.all(q8[0, 0, 4] == 0) and qs[0, 0, 4] == F32(F32(F32(1e-12) / F32(127)) / F32(128))


def test_rotation_by_head_dim():
    """head_dim 256 rotates each 128-channel half by H128 (block-diagonal, x @ diag(H, H)); 96 is not rotated;
    64 / 128 use the full-order matrix.  Integer rows keep every float64 sum exact, so equality is exact."""
    rng = np.random.default_rng(9)
    for d, rb in ((64, 64), (96, 0), (128, 128), (256, 128)):
        assert orc.rotation_block(d) == rb
        x = rng.integers(-40, 40, size=(5, d)).astype(np.float64)
        if rb == 0:
            expect = x
        else:
            h = orc.hadamard_pm1(rb)
            expect = np.concatenate([x[:, i:i + rb] @ h for i in range(0, d, rb)], axis=1)
        assert np.array_equal(orc.rotate_rows(x), expect), d


@pytest.mark.parametrize("d", [96, 256])
def test_quant_q_invariants_other_head_dims(d):
    """QS = s / RB with RB = 128 for d256 (each block multiplies its share of Q K^T by 128), QS = s for d96."""
    q = _bf16((1, 2, 70, d), 60 + d)
    q8, qs = orc.quant_q(q)
    x = orc.rotate_rows(q).astype(F32)
    amax = np.abs(x).max(-1)
    assert np.all(np.abs(q8.astype(int)).max(-1) == 127)
    s = qs * (128 if d == 256 else 1)
    assert np.allclose(s * 127, amax, rtol=1e-6)
    if d == 96:
        assert np.allclose(s * 127, np.abs(q).max(-1), rtol=1e-6)   # the raw row's max: no rotation
    assert np.all(np.abs(q8 * s[..., None] - x) <= s[..., None] * 0.5 * (1 + 1e-5))
    # the scores the kernel sees: Q8 K8^T * QS * KS equals Q K^T up to quantization error, for both head dims
    k = _bf16((1, 2, 64, d), 61 + d)
    k8, ks, _, _ = orc.quant_kv(k, k)
    sc = (q8.astype(np.float64) @ np.swapaxes(k8, -1, -2).astype(np.float64)) * qs[..., None] * np.repeat(ks, 32, -1)[:, :, None, :64]
    ref = q.astype(np.float64) @ np.swapaxes(k, -1, -2).astype(np.float64)
    assert np.abs(sc - ref).max() <= 0.02 * np.abs(ref).max()


@pytest.mark.parametrize("d,causal", [(96, False), (96, True), (256, False), (256, True)])
def test_emulation_other_head_dims_vs_float64(d, causal):
    q, k, v = _bf16((1, 2, 200, d), 70 + d), _bf16((1, 2, 200, d), 71 + d), _bf16((1, 2, 200, d), 72 + d)
    out = orc.sage_forward(q, k, v, causal=causal, block_n=64)
    assert _cos(out, orc.sdpa_reference(q, k, v, causal=causal)) >= 0.999


def test_quant_kv_invariants_and_vector_norm():
    k = _bf16((1, 2, 100, 64), 7)
    v = _bf16((1, 2, 100, 64), 8, 3.0)
    v[:, :, :, 5] = 0.0
    k8, ks, v8, vs = orc.quant_kv(k, v, seq_pad=128)
    # VS is torch.linalg.vector_norm(v, inf, dim=seq, dtype=float32), the reference's own op (_attention.py:121)
    ref_vs = torch.linalg.vector_norm(torch.from_numpy(v).to(torch.bfloat16), ord=float("inf"), dim=2,
                                      dtype=torch.float32).numpy()
    assert np.array_equal(vs, ref_vs)
    assert k8.shape == (1, 2, 128, 64) and ks.shape == (1, 2, 4)
    assert np.all(k8[:, :, 100:] == 0) and np.all(v8[:, :, 100:] == 0)   # pad rows are zero
    blk = np.abs(k8.astype(int)).reshape(1, 2, 4, 32, 64).max(axis=(-1, -2))
    assert np.all(blk == 127)                                         # each 32-key block spans the int8 range
    x = orc.fwht_rows(k).astype(F32)
    # KS is max|x| / 127 of the block and is NOT divided by the rotation order (sage_quant.py:63-66)
    assert np.allclose(ks[:, :, 0] * 127, np.abs(x[:, :, :32]).max(axis=(-1, -2)), rtol=1e-6)
    dec = orc.e4m3_to_f32(v8[:, :, :100])
    assert np.all(dec[..., 5] == 0)                                   # zero channel stays zero
    am = np.abs(v).argmax(axis=2)
    for c in (0, 7, 63):                                              # each channel's amax element maps to +-448
        assert abs(dec[0, 0, am[0, 0, c], c]) == 448.0
    rel = np.abs(dec * vs[:, :, None, :] / 448 - v) / np.maximum(np.abs(v), 1e-3)
    assert np.all(rel[np.abs(v) > vs[:, :, None, :] / 16] <= 2.0 ** -4 + 1e-6)   # E4M3: 3 mantissa bits


# ------------------------------------------------------------------------------------------------ attention
def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float((a * b).sum() / math.sqrt((a * a).sum() * (b * b).sum()))


@pytest.mark.parametrize("block_n", [32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_emulation_vs_float64_attention(block_n, causal):
    """Config-1-like shape on CPU: the quantized path stays within the reference's accuracy (cos ~0.9992)."""
    q, k, v = _bf16((1, 4, 512, 64), 9), _bf16((1, 4, 512, 64), 10), _bf16((1, 4, 512, 64), 11)
    out = orc.sage_forward(q, k, v, causal=causal, block_n=block_n)
    assert _cos(out, orc.sdpa_reference(q, k, v, causal=causal)) >= 0.999


def test_emulation_single_key_returns_dequantized_v():
    """One key: p = exp2(arg) with arg = 0 up to the two roundings of nk = neg - fp32(c * 2^26 * ct) (c = 1 / (2 pi),
    the kernel's seed), each at most half an ulp of ~c * 2^26 * ct <= 0.75 * ct.  So out = dequantized V / p with
    |p - 1| <= 2^(1.5 ct) - 1 (the
    E4M3 cast of p is exactly 1), and nothing else may perturb it."""
    q, k, v = _bf16((1, 2, 5, 128), 12), _bf16((1, 2, 1, 128), 13), _bf16((1, 2, 1, 128), 14)
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v)
    out = orc.attention(q8, qs, k8, ks, v8, vs, 1, out_dtype="f32")
    deq = orc.e4m3_to_f32(v8[:, :, :1]) * vs[:, :, None, :] / 448.0
    ct = orc.logit_scale_base(128).astype(np.float64) * qs * ks[:, :, :1]          # [B, H, Sq]
    bound = np.exp2(1.51 * ct) - 1.0 + 1e-6
    rel = np.abs(out / np.broadcast_to(deq, out.shape) - 1.0).max(axis=-1)
    assert (rel <= bound).all(), (rel.max(), bound.min())
    assert bound.max() < 1e-3



def test_emulation_large_scales_read_scores_exactly(monkeypatch):
    """Inputs scaled by 100: the seeded read's offset rounding (up to ~1.5 ct log2 units, ct the logit per unit of S)
    would move a single key's p far from 1, so the rule reads such groups exactly (F - c) with the reference's
    offset, arg = fp32(S * fp32(cl * ks) - fp32(cl * fp32(S * ks))), |arg| <= 3.1 * 2^-24 * |logit|.  At scale 1
    the rule does not fire.  Planted mistake: without the rule (CT_WIDE = inf) the same bound fails."""
    def run(scale):
        q = _bf16((1, 2, 5, 64), 60) * scale
        k = _bf16((1, 2, 1, 64), 61) * scale
        v = _bf16((1, 2, 1, 64), 62)
        q, k = orc.round_to_bf16(q), orc.round_to_bf16(k)
        q8, qs = orc.quant_q(q)
        k8, ks, v8, vs = orc.quant_kv(k, v)
        cl = (orc.logit_scale_base(64) * qs).astype(np.float32)
        wide = orc.wide_rows(cl, ks, 1, np.arange(5), np.arange(2))
        out = orc.attention(q8, qs, k8, ks, v8, vs, 1, out_dtype="f32")
        deq = orc.e4m3_to_f32(v8[:, :, :1]) * vs[:, :, None, :] / 448.0
        s = np.matmul(q8.astype(np.float64), np.swapaxes(k8[:, :, :1].astype(np.float64), -1, -2))[..., 0]
        logit = np.abs(s * cl.astype(np.float64) * ks[:, :, :1].astype(np.float64))            # [B, H, Sq]
        bound = np.exp2(3.1 * 2.0 ** -24 * logit) - 1.0 + 1e-6
        rel = np.abs(out / np.broadcast_to(deq, out.shape) - 1.0).max(axis=-1)
        return wide, rel, bound
    wide, rel, bound = run(1.0)
    assert not wide.any()
    wide, rel, bound = run(100.0)
    assert wide.all() and np.isfinite(rel).all()
    assert (rel <= bound).all(), (rel.max(), bound.min())
    assert bound.max() < 0.02
    monkeypatch.setattr(orc, "CT_WIDE", float("inf"))
    wide, rel, bound = run(100.0)
    assert not wide.any()
    assert not (rel <= bound).all()

def test_emulation_causal_first_row_and_bottom_right():
    q, k, v = _bf16((1, 1, 40, 64), 15), _bf16((1, 1, 40, 64), 16), _bf16((1, 1, 40, 64), 17)
    out = orc.sage_forward(q, k, v, causal=True, block_n=32, out_dtype="f32")
    k8, ks, v8, vs = orc.quant_kv(k, v)
    deq0 = orc.e4m3_to_f32(v8[0, 0, 0]) * vs[0, 0] / 448.0
    # row 0 sees key 0 only: dequantized V up to p = 2^arg, |arg| <= 1.5 ct (see the single-key test)
    q8, qs = orc.quant_q(q)
    ct0 = float(orc.logit_scale_base(64)) * float(qs[0, 0, 0]) * float(ks[0, 0, 0])
    assert np.abs(out[0, 0, 0] / deq0 - 1.0).max() <= np.exp2(1.51 * ct0) - 1.0 + 1e-6
    # each row only depends on keys <= its index: changing the last key (in its own 32-key block, so no K scale
    # of an earlier block moves) leaves every row of the first 32 unchanged
    k2 = k.copy()
    k2[..., -1, :] += 3.0
    out2 = orc.sage_forward(q, k2, v, causal=True, block_n=32, out_dtype="f32")
    assert np.array_equal(out[..., :32, :], out2[..., :32, :])
    assert not np.array_equal(out[..., 39, :], out2[..., 39, :])


def test_emulation_causal_q_longer_than_kv():
    """Bottom-right causal with q_len > kv_len: row i sees keys <= i - (q_len - kv_len).  Rows that see no key are 0
    (the gfx950 convention), and every other row equals the same query's row of the q_len == kv_len call on the last
    kv_len queries, bit for bit (per-token Q scales and per-row softmax state do not depend on the other rows)."""
    q, k, v = _bf16((1, 2, 70, 64), 40), _bf16((1, 2, 40, 64), 41), _bf16((1, 2, 40, 64), 42)
    out = orc.sage_forward(q, k, v, causal=True, block_n=64, out_dtype="f32")
    assert np.isfinite(out).all()
    assert (out[:, :, :30] == 0).all()
    tail = orc.sage_forward(np.ascontiguousarray(q[:, :, 30:]), k, v, causal=True, block_n=64, out_dtype="f32")
    assert np.array_equal(out[:, :, 30:], tail)
    ref = orc.sdpa_reference(q[:, :, 30:], k, v, causal=True)
    assert _cos(out[:, :, 30:], ref) >= 0.999


def test_emulation_causal_q_shorter_than_kv():
    """q_len < kv_len: query i sees keys <= i + (kv_len - q_len), i.e. it is row i + kv_len - q_len of the square
    causal call whose last q_len queries are these, bit for bit."""
    q_all, k, v = _bf16((1, 2, 50, 64), 43), _bf16((1, 2, 50, 64), 44), _bf16((1, 2, 50, 64), 45)
    q = np.ascontiguousarray(q_all[:, :, 30:])
    out = orc.sage_forward(q, k, v, causal=True, block_n=64, out_dtype="f32")
    full = orc.sage_forward(q_all, k, v, causal=True, block_n=64, out_dtype="f32")
    assert np.array_equal(out, full[:, :, 30:])
    assert not np.array_equal(out, orc.sage_forward(q, k, v, causal=False, block_n=64, out_dtype="f32"))


def test_varlen_oracle_sequences_and_edge_rows():
    """Packed batch with an empty query sequence, a sequence without keys and a causal sequence longer than its keys:
    each sequence is its own call (pinned against float64 attention), rows outside every sequence stay NaN."""
    H, Hkv, D = 4, 2, 64
    cu_q = np.array([0, 37, 37, 100, 131, 160])
    cu_k = np.array([0, 90, 150, 150, 170, 260])
    q = _bf16((170, H, D), 46)       # rows 160.. belong to no sequence
    k, v = _bf16((260, Hkv, D), 47), _bf16((260, Hkv, D), 48)
    for causal in (False, True):
        out = orc.sage_forward_varlen(q, k, v, cu_q, cu_k, causal=causal)
        assert np.isnan(out[160:]).all() and np.isfinite(out[:160]).all()
        assert (out[37:100] == 0).all()                              # sequence 2 has no keys
        hnd = lambda t: np.ascontiguousarray(t.transpose(1, 0, 2))[None]   # noqa: E731
        seqs = ((0, 37, 0, 90), (131, 160, 170, 260)) + (() if causal else ((100, 131, 150, 170),))
        for (q0, q1, k0, k1) in seqs:
            ref = orc.sdpa_reference(hnd(q[q0:q1]), hnd(k[k0:k1]), hnd(v[k0:k1]), causal=causal)[0].transpose(1, 0, 2)
            assert _cos(out[q0:q1], ref) >= 0.999
        if causal:   # sequence 3: 31 queries, 20 keys: the first 11 rows see no key
            assert (out[100:111] == 0).all() and (out[111:131] != 0).any(axis=(1, 2)).all()


def test_emulation_softmax_bookkeeping_gives_exact_lse():
    """The running max / lazy rescale / running sum must reproduce the logsumexp of the quantized logits
    S * QS * KS * sm computed directly; this fails for a dropped correction term or a misplaced K scale."""
    q, k, v = _bf16((1, 2, 64, 128), 18), _bf16((1, 2, 300, 128), 19, 2.0), _bf16((1, 2, 300, 128), 20)
    k[:, :, 100:140] *= 8.0                      # blocks with very different K scales
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v)
    for bn in (32, 64):
        _, m, l = orc.attention(q8, qs, k8, ks, v8, vs, 300, block_n=bn, return_stats=True)
        cl = orc.logit_scale_base(128) * qs
        lse2 = cl.astype(np.float64) * m + np.log2(l.astype(np.float64))
        ksr = np.repeat(ks, 32, axis=-1)[:, :, :300]
        s = np.einsum("bhqd,bhkd->bhqk", q8.astype(np.float64), k8[:, :, :300].astype(np.float64))
        logit2 = s * cl[..., None].astype(np.float64) * ksr[:, :, None, :]
        mx = logit2.max(-1)
        exact = mx + np.log2(np.exp2(logit2 - mx[..., None]).sum(-1))
        # every exponent argument is within 1.5 ct + 2^-24 |cl m| of S ct - cl m: nk = neg - fp32(c * 2^26 * ct)
        # rounds twice, each time by at most half an ulp of ~c * 2^26 * ct <= 0.75 ct; the logsumexp moves by at
        # most that
        ct_max = (cl[..., None].astype(np.float64) * ks[:, :, None, :]).max(-1)
        bound = 1.51 * ct_max + 2.0 ** -23 * np.abs(cl * m) + 2e-5
        assert (np.abs(lse2 - exact) <= bound).all(), bn
        assert bound.max() < 5e-3


def test_split_emulation_gives_exact_lse_and_matches_unsplit():
    """Split-key-range merge (the gfx950 kernel's tail tiles): the merged (M, L) must still give the logsumexp (a
    wrong merge weight or sign fails), one chunk must equal the unsplit emulation up to the fp16 rounding of the
    stored O / l, and the merged output must stay as close to float64 attention as the unsplit one."""
    q, k, v = _bf16((1, 2, 64, 128), 18), _bf16((1, 2, 300, 128), 19, 2.0), _bf16((1, 2, 300, 128), 20)
    k[:, :, 100:140] *= 8.0
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v)
    rows = np.ones((1, 2, 64), dtype=bool)
    rows[:, 1, 32:] = False                       # unsplit rows must come back untouched
    base, m0, l0 = orc.attention(q8, qs, k8, ks, v8, vs, 300, block_n=64, out_dtype="f32", return_stats=True)
    one = orc.attention(q8, qs, k8, ks, v8, vs, 300, block_n=64, out_dtype="f32", kv_split=(1, rows))
    # one chunk: the same online softmax, with O passed through fp16(O / l) (relative rounding <= 2^-11)
    assert np.array_equal(one[~rows], base[~rows])
    assert (np.abs(one - base) <= 2.0 ** -10 * np.abs(base) + 1e-6).all()
    assert not np.array_equal(one[rows], base[rows])
    cl = orc.logit_scale_base(128) * qs
    ksr = np.repeat(ks, 32, axis=-1)[:, :, :300]
    s = np.einsum("bhqd,bhkd->bhqk", q8.astype(np.float64), k8[:, :, :300].astype(np.float64))
    logit2 = s * cl[..., None].astype(np.float64) * ksr[:, :, None, :]
    mx = logit2.max(-1)
    exact = mx + np.log2(np.exp2(logit2 - mx[..., None]).sum(-1))
    ref = orc.sdpa_reference(q, k, v)
    ct_max = (cl[..., None].astype(np.float64) * ks[:, :, None, :]).max(-1)
    for chunks in (2, 3, 5):
        out, m, l = orc.attention(q8, qs, k8, ks, v8, vs, 300, block_n=64, out_dtype="f32", return_stats=True,
                                  kv_split=(chunks, rows))
        lse2 = cl.astype(np.float64) * m + np.log2(l.astype(np.float64))
        # the bound of the unsplit bookkeeping test (exponent arguments within 1.5 ct of exact)
        assert (np.abs(lse2 - exact) <= 1.51 * ct_max + 2.0 ** -23 * np.abs(cl * m) + 2e-5).all(), chunks
        assert np.array_equal(out[~rows], base[~rows]) and np.array_equal(m[~rows], m0[~rows])
        # the split keeps small probabilities that an unsplit tile flushes in E4M3, so it is compared with float64
        # attention, not with the unsplit emulation
        assert _cos(out, ref) >= _cos(base, ref) - 1e-4, chunks
    # O and L must be merged with the same weights: with V = 1 every output is sum(p8) / sum(p) ~ 1
    ones = np.ones_like(v)
    k8, ks, v8, vs = orc.quant_kv(_bf16((1, 2, 300, 128), 19), ones)
    for chunks in (2, 3, 5):
        out = orc.attention(q8, qs, k8, ks, v8, vs, 300, block_n=64, out_dtype="f32", kv_split=(chunks, rows))
        assert np.abs(out - 1.0).max() < 1e-2, chunks


def _walk_inputs(kind, sq, skv, seed):
    """One head of HunyuanVideo-like (N(0, 0.5^2), a shared K channel bias ~ N(0, 2)) or Wan-like (N(0, 1), 3 channels
    x10 in K and in V) inputs, bf16 values as float32 [1, 1, S, 128]."""
    g = torch.Generator().manual_seed(seed)
    if kind == "wan":
        q, k, v = (torch.randn(1, 1, s, 128, generator=g) for s in (sq, skv, skv))
        k[..., torch.randperm(128, generator=g)[:3]] *= 10.0
        v[..., torch.randperm(128, generator=g)[:3]] *= 10.0
    else:
        q, k, v = (torch.randn(1, 1, s, 128, generator=g) * 0.5 for s in (sq, skv, skv))
        k += torch.randn(128, generator=g) * math.sqrt(2.0)
    return [t.to(torch.bfloat16).float().numpy() for t in (q, k, v)]


@pytest.mark.parametrize("kind,chunks,max_gap", [
    ("flux", 8, 2e-3),          # Flux (config 2) head 22: 96 split tiles x 8 key ranges on a 256-CU MI355X
    ("hunyuan", 2, 5e-4),       # HunyuanVideo-like, 2 ranges as config 4's plan
    ("wan", 3, None),           # Wan-like x10 outlier channels, 3 ranges as config 3's plan
])
def test_split_ranges_stay_near_the_reference_walk(kind, chunks, max_gap):
    """The gfx950 kernel splits the key range of the short last round's query tiles into contiguous ranges, merged
    afterwards (no counterpart in the reference, which walks every key of a tile in one online softmax:
    kernel_build/make_sage_r2.py:141-253).  Ranges after the first start from the walk's running max after the
    first key tile, so wherever the walk's max stays put after that tile they form the walk's own probabilities and
    E4M3 bytes.  Flux (every third query tile of head 22, the benchmark inputs) and HunyuanVideo-like inputs stay
    within a few output ulps of the walk (measured max 4.9e-4 over all of Flux head 22 and 1.2e-4; ranges started
    from -inf gave 6.1e-3 and 2.3e-4) with > 85% of the elements bit-identical.  Wan's x10 outlier channels move the
    walk's max after its first tile, and where they do the split keeps small probabilities that the walk's E4M3
    flushes: there the gap (measured 0.13-0.16 at outputs up to ~6) stays below the walk's own distance to float64
    attention (0.31-0.53), the mean gap below a fifth of the walk's mean error, and the split rows are no further
    from float64 attention than the walk."""
    if kind == "flux":
        from cdna4_sage.configs import CONFIGS, make_inputs

        cfg = CONFIGS["2"]
        q, k, v = make_inputs(cfg, heads=slice(22, 23))
        qn, kn, vn = (t.float().numpy() for t in (q, k, v))
        rows = np.concatenate([np.arange(t * 128, t * 128 + 128) for t in range(0, 36, 3)])
        skv = cfg.S
    else:
        qn, kn, vn = _walk_inputs(kind, 384, 8192, seed=1)
        skv = 8192
        rows = np.arange(384) + skv - 384
        qn = np.concatenate([np.zeros((1, 1, skv - 384, 128), F32), qn], axis=2)   # the rows' positions
    q8, qs = orc.quant_q(np.ascontiguousarray(qn[:, :, rows]))
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=(skv + 127) // 128 * 128)
    split = (chunks, np.ones((1, 1, len(rows)), dtype=bool))
    out, walk = orc.attention(q8, qs, k8, ks, v8, vs, skv, block_n=32, kv_split=split, q_rows=rows, seq_q=skv,
                              also_unsplit=True)
    ref = orc.sdpa_reference(np.ascontiguousarray(qn[:, :, rows]), kn, vn)
    gap = np.abs(out - walk)
    own = np.abs(walk - ref)                      # the reference walk's own distance to float64 attention
    assert not np.array_equal(out, walk)          # the split does change bits: the check is not vacuous
    assert float((out == walk).mean()) >= 0.85 if max_gap is not None else float((out == walk).mean()) >= 0.8
    if max_gap is not None:
        assert float(gap.max()) <= max_gap, float(gap.max())
    assert float(gap.max()) <= float(own.max()), (float(gap.max()), float(own.max()))
    assert float(gap.mean()) <= 0.2 * float(own.mean())
    assert _cos(out, ref) >= _cos(walk, ref) - 1e-5
    # the unseeded split (every range from -inf) is the farther one: the seed is what brings the ranges to the walk
    if max_gap is not None:
        cl = (orc.logit_scale_base(128) * qs).astype(F32)
        assert float(np.abs(_split_from_minus_inf(q8, cl, k8, ks, v8, vs, skv, chunks, rows) - walk).max()) > max_gap


def test_split_range_whose_probabilities_underflow_against_the_seed():
    """A range that starts from the seeded max can hold only probabilities far below it: with key 0 leading every
    other key by 124-152 in the exponent, each later range of the 4-range split has l in (0, 2^-128) on 72 of the 128
    rows (l = 0 on 14) and O = 0 (every E4M3 byte of P is 0).  1 / l overflows there; the stored partial must still
    be 0 (l and O scaled by 2^64 before the reciprocal), not 0 * inf = NaN, and the merge must give the walk's output
    (V of key 0) up to the fp16 rounding of the first range's O / l (one bf16 step of outputs up to ~4)."""
    from gpu_util import underflow_split_inputs

    q, k, v = underflow_split_inputs()
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v, seq_pad=1024)
    out, walk = orc.attention(q8, qs, k8, ks, v8, vs, 1024, block_n=32, kv_split=(4, np.ones((1, 1, 128), bool)),
                              also_unsplit=True)
    assert np.isfinite(out).all()
    assert float(np.abs(out - walk).max()) <= 2.0 ** -6
    assert float(np.abs(walk - orc.sdpa_reference(q, k, v)).max()) <= 0.1
    # the case does reach the overflow: some range has 0 < l < 2^-128 after the seeded start
    cl = (orc.logit_scale_base(128) * qs).astype(F32)
    rows = (np.arange(128), 128)
    wide = orc.wide_rows(cl, ks, 1024, rows[0], np.arange(1))
    _, m_seed = orc._seed_tiles(q8, cl, k8, ks, v8, 1024, False, 32, orc.RESCALE_THRESHOLD, None, rows, wide)
    o, _, l = orc._online_softmax(q8, cl, k8, ks, v8, 1024, False, 32, orc.RESCALE_THRESHOLD, 8, 16, None, rows, wide,
                                  m_init=m_seed)
    assert int(((l > 0) & (l < F32(2.0 ** -128))).sum()) > 0 and not o.any()


def _split_from_minus_inf(q8, cl, k8, ks, v8, vs, seq_kv, chunks, rows):
    """The merged split with every range's softmax from m = -inf (the previous kernel's split; bf16 output)."""
    qpos = (rows, seq_kv)
    hk = np.arange(q8.shape[1]) // (q8.shape[1] // k8.shape[1])
    wide = orc.wide_rows(cl, ks, seq_kv, rows, hk)
    kt = (seq_kv + 63) // 64
    parts = [orc._online_softmax(q8, cl, k8, ks, v8, seq_kv, False, 32, orc.RESCALE_THRESHOLD, c * kt // chunks * 2,
                                 (c + 1) * kt // chunks * 2, None, qpos, wide) for c in range(chunks)]
    mm = np.max([p[1] for p in parts], axis=0)
    ll = np.zeros_like(parts[0][2])
    oo = np.zeros_like(parts[0][0])
    for oc, mc, lc in parts:
        w = (np.exp2(((mc - mm) * cl).astype(F32)).astype(F32) * lc).astype(F32)
        ll = (ll + w).astype(F32)
        oo = (oo + (w[..., None] * (oc / lc[..., None]).astype(F32).astype(np.float16).astype(F32))).astype(F32)
    out = ((oo * (F32(1.0 / 448.0) / ll)[..., None]).astype(F32) * vs[:, hk][:, :, None, :]).astype(F32)
    return orc.round_output(out, "bf16")


def test_mask_identities():
    """Boolean attn_mask pins: an all-True mask is no mask; the bottom-right triangle as a mask is the causal flag; a
    key-padding mask equals the call on the shorter key range with the same quantized K / V (per-row softmax state
    never sees a masked key); a row whose mask is all False is 0 (and no NaN reaches the other rows)."""
    q, k, v = _bf16((2, 3, 90, 64), 60), _bf16((2, 3, 150, 64), 61), _bf16((2, 3, 150, 64), 62)
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v)
    base = orc.attention(q8, qs, k8, ks, v8, vs, 150, block_n=64, out_dtype="f32")
    allt = orc.attention(q8, qs, k8, ks, v8, vs, 150, block_n=64, out_dtype="f32", attn_mask=np.ones((150,), bool))
    assert np.array_equal(base, allt)
    causal = orc.attention(q8, qs, k8, ks, v8, vs, 150, causal=True, block_n=64, out_dtype="f32")
    tri = np.arange(150)[None, :] <= np.arange(90)[:, None] + 60
    assert np.array_equal(causal, orc.attention(q8, qs, k8, ks, v8, vs, 150, block_n=64, out_dtype="f32",
                                                attn_mask=tri))
    # causal flag and a mask together: the AND of both
    half = np.arange(150) % 2 == 0
    assert np.array_equal(orc.attention(q8, qs, k8, ks, v8, vs, 150, causal=True, block_n=64, out_dtype="f32",
                                        attn_mask=half),
                          orc.attention(q8, qs, k8, ks, v8, vs, 150, block_n=64, out_dtype="f32",
                                        attn_mask=tri & half))
    for n in (1, 64, 100):          # one key, a whole tile, a partial tile
        pad = np.arange(150)[None, None, None, :] < n
        short = orc.attention(q8, qs, k8, ks, v8, vs, n, block_n=64, out_dtype="f32")
        assert np.array_equal(short, orc.attention(q8, qs, k8, ks, v8, vs, 150, block_n=64, out_dtype="f32",
                                                   attn_mask=pad)), n
    rowmask = np.ones((2, 1, 90, 150), bool)
    rowmask[1, :, 7] = False
    out = orc.attention(q8, qs, k8, ks, v8, vs, 150, block_n=64, out_dtype="f32", attn_mask=rowmask)
    assert np.isfinite(out).all() and (out[1, :, 7] == 0).all()
    assert np.array_equal(np.delete(out, 7, axis=2), np.delete(base, 7, axis=2))


def test_masked_emulation_vs_float64_and_split():
    """A random mask (a third of the keys hidden, per batch, head and row), with and without the causal flag: the
    quantized path stays within the accuracy of the unmasked one against the float64 masked softmax, and split key
    ranges (including ranges in which a row sees no key, and rows that see no key at all) merge to the unsplit
    result up to the fp16 rounding of the stored O / l."""
    rng = np.random.default_rng(63)
    q, k, v = _bf16((1, 2, 70, 128), 64), _bf16((1, 2, 260, 128), 65), _bf16((1, 2, 260, 128), 66)
    mask = rng.random((1, 2, 70, 260)) > 0.33
    mask[0, 0, 5, :] = False                         # a row that sees nothing
    mask[0, 1, 9, :] = False
    mask[0, 1, 9, 250] = True                        # a row that sees one key of the last tile only
    for causal in (False, True):
        out = orc.sage_forward(q, k, v, causal=causal, block_n=64, out_dtype="f32", attn_mask=mask)
        ref = orc.sdpa_reference(q, k, v, causal=causal, attn_mask=mask)
        assert np.isfinite(out).all() and (out[0, 0, 5] == 0).all() and (ref[0, 0, 5] == 0).all()
        assert _cos(out, ref) >= 0.999, causal
        rows = np.ones((1, 2, 70), dtype=bool)
        for chunks in (2, 5):
            sp = orc.sage_forward(q, k, v, causal=causal, block_n=64, out_dtype="f32", attn_mask=mask,
                                  kv_split=(chunks, rows))
            assert np.isfinite(sp).all() and (sp[0, 0, 5] == 0).all()
            assert _cos(sp, ref) >= _cos(out, ref) - 1e-4, (causal, chunks)
            # row 9 of head 1 sees one key, in the last range: the merge must return that range alone
            assert np.abs(sp[0, 1, 9] - out[0, 1, 9]).max() <= 2.0 ** -10 * np.abs(out[0, 1, 9]).max() + 1e-6


def test_float_mask_identities_and_bias_path():
    """Additive (float) masks.  All zero: no mask, bit for bit (every tile takes the boolean path).  Values 0 / -inf:
    the boolean mask, bit for bit.  A constant per row (softmax is shift-invariant): the unmasked result up to the
    rounding of the bias path, which a wrong log2(e) factor, a bias left out of the row max or a wrong rescale of m
    would break.  An ALiBi-style bias: float64 attention with the same bias.  Split ranges merge the bias path."""
    rng = np.random.default_rng(70)
    q, k, v = _bf16((1, 2, 70, 64), 71), _bf16((1, 2, 200, 64), 72), _bf16((1, 2, 200, 64), 73)
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v)
    att = lambda **kw: orc.attention(q8, qs, k8, ks, v8, vs, 200, block_n=64, out_dtype="f32", **kw)  # noqa: E731
    base = att()
    assert np.array_equal(att(attn_mask=np.zeros((70, 200), np.float32)), base)
    boolm = rng.random((1, 2, 70, 200)) > 0.4
    fm = np.where(boolm, np.float32(0), np.float32(-np.inf))
    assert np.array_equal(att(attn_mask=fm), att(attn_mask=boolm))
    for c in (3.0, -7.5, 40.0):
        shifted = att(attn_mask=np.full((1, 2, 70, 1), c, np.float32) * np.ones((1, 1, 1, 200), np.float32))
        assert np.abs(shifted - base).max() <= 1e-2 and _cos(shifted, base) >= 0.9999, c
    wrong = att(attn_mask=np.tile(np.arange(200, dtype=np.float32) * 0.01, (70, 1)))
    assert not np.array_equal(wrong, base)
    slope = np.float32(0.05)
    alibi = (-slope * np.abs(np.arange(70)[:, None] + 130 - np.arange(200)[None, :])).astype(np.float32)
    alibi = orc.round_to_bf16(alibi)
    for causal in (False, True):
        out = att(attn_mask=alibi, causal=causal)
        ref = orc.sdpa_reference(q, k, v, causal=causal, attn_mask=alibi)
        assert _cos(out, ref) >= 0.999, causal
        # the bias changes the result: the unbiased call is further from the biased reference
        assert _cos(att(causal=causal), ref) < _cos(out, ref)
    mixed = alibi.copy()
    mixed[5] = -np.inf                         # a row that sees nothing
    mixed[9, :150] = -np.inf                   # a row that sees only the last 50 keys
    out = att(attn_mask=mixed)
    assert np.isfinite(out).all() and (out[:, :, 5] == 0).all()
    ref = orc.sdpa_reference(q, k, v, attn_mask=mixed)
    assert _cos(out, ref) >= 0.999
    rows = np.ones((1, 2, 70), dtype=bool)
    sp = att(attn_mask=mixed, kv_split=(3, rows))
    assert np.isfinite(sp).all() and (sp[:, :, 5] == 0).all() and _cos(sp, ref) >= _cos(out, ref) - 1e-4


def test_split_rows_numbering():
    r = orc.split_rows(2, 3, 300, n_full=7)          # q_tiles = 3: tile = (b * 3 + h) * 3 + row // 128
    assert r.shape == (2, 3, 300)
    assert not r[0, 2, 0] and r[0, 2, 128] and r[1].all()   # tile 6 whole, tile 7 split, batch 1 all split
    s = orc.split_rows(2, 3, 300, n_full=7, heads=[2])
    assert np.array_equal(s[:, 0], r[:, 2])


def test_emulation_gqa_equals_repeated_heads():
    q, k, v = _bf16((1, 4, 70, 64), 21), _bf16((1, 1, 90, 64), 22), _bf16((1, 1, 90, 64), 23)
    a = orc.sage_forward(q, k, v, block_n=64)
    b = orc.sage_forward(q, np.repeat(k, 4, 1), np.repeat(v, 4, 1), block_n=64)
    assert np.array_equal(a, b)


def test_v8_device_layout_permutation():
    v8 = np.random.default_rng(24).integers(0, 256, (1, 2, 128, 64)).astype(np.uint8)
    t = orc.v8_to_device_layout(v8)
    for key in range(128):
        grp, g, h, r = key // 64, (key % 64) // 8, (key // 4) % 2, key % 4
        assert np.array_equal(t[:, :, :, 64 * grp + 32 * h + 4 * g + r], v8[:, :, key, :])
    assert np.array_equal(orc.v8_from_device_layout(t), v8)


def test_lse_reference_matches_torch_logsumexp():
    q, k = _bf16((1, 2, 50, 64), 25), _bf16((1, 2, 80, 64), 26)
    for causal in (False, True):
        got = orc.lse_reference(q, k, causal=causal)
        sc = torch.from_numpy(q).double() @ torch.from_numpy(k).double().transpose(-1, -2) * 64 ** -0.5
        if causal:
            sc.masked_fill_(torch.ones(50, 80, dtype=torch.bool).tril(80 - 50).logical_not(), float("-inf"))
        assert np.allclose(got, torch.logsumexp(sc, -1).numpy(), atol=1e-10)


# ---------------------------------------------------------------------------------------------------------------
# The lazy rescale and the E4M3 probabilities, on hand-made quantized operands (one query, 64 keys, head dim 64):
# q8 = e_0, k8[j] = s_j e_0, so S_j = s_j; KS = 1 and QS chosen so that cl = fp32(1/8): key j's logit is s_j / 8
# in log2 units.  V is one-hot (key j -> channel j, V8 = 448, VS = 1), so out_c * l = p8_c, the E4M3 probability
# the PV product used for key c.
# ---------------------------------------------------------------------------------------------------------------
CL_HANDMADE = 1.0 / 8


def _handmade(s_keys):
    d = 64
    q8 = np.zeros((1, 1, 1, d), dtype=np.int8)
    q8[..., 0] = 1
    k8 = np.zeros((1, 1, d, d), dtype=np.int8)
    k8[0, 0, :, 0] = np.asarray(s_keys, dtype=np.int64)
    ks = np.ones((1, 1, 2), dtype=np.float32)
    qs = np.full((1, 1, 1), np.float32(CL_HANDMADE) / orc.logit_scale_base(d), dtype=np.float32)
    v8 = np.zeros((1, 1, d, d), dtype=np.uint8)
    v8[0, 0, np.arange(d), np.arange(d)] = orc.f32_to_e4m3(np.array([448.0], dtype=np.float32))[0]
    vs = np.ones((1, 1, d), dtype=np.float32)
    return q8, qs, k8, ks, v8, vs


def _p8(s_keys, **kw):
    q8, qs, k8, ks, v8, vs = _handmade(s_keys)
    out, m, l = orc.attention(q8, qs, k8, ks, v8, vs, 64, out_dtype="f32", return_stats=True, **kw)
    return out[0, 0, 0].astype(np.float64) * float(l[0, 0, 0]), float(m[0, 0, 0])


def test_lazy_rescale_keeps_stale_max_below_threshold_and_moves_above():
    """Block 0's max sets m (key 0, logit 1); block 1's key 40 rises by 5 log2 units: below the threshold of 8
    (make_sage_r2.py:185-187) the max stays stale, so key 40's probability is 2^5 and enters the PV product as
    E4M3(32) = 32; a rise of 10 moves the max to key 40 (probability 1).  A threshold other than 8 between 5 and 10,
    or a decision over the 64-key tile instead of per 32-key block, fails one of the two."""
    s = np.zeros(64, dtype=np.int64)
    s[0] = 8
    s[40] = 8 * 6
    p8, m = _p8(s)
    assert m == 8.0                                    # stale: block 0's max (S * KS units)
    assert abs(p8[40] - 32.0) < 1e-4 and abs(p8[0] - 1.0) < 1e-6
    s[40] = 8 * 11
    p8, m = _p8(s)
    assert m == 88.0                                   # moved to key 40
    assert abs(p8[40] - 1.0) < 1e-6
    # the per-block decision is what keeps the max stale: one decision over the 64-key tile moves it at once
    s[40] = 8 * 6
    p8_64, m64 = _p8(s, block_n=64)
    assert m64 == 48.0 and abs(p8_64[40] - 1.0) < 1e-6


def test_probabilities_entering_pv_are_e4m3():
    """Every probability that reaches the PV product is an E4M3 value (make_sage_r2.py:208-214 pack P to fp8); the
    float probabilities of these keys are not, so an emulation that dropped the rounding fails."""
    rng = np.random.default_rng(5)
    s = rng.integers(-60, 61, size=64)
    p8, m = _p8(s)
    e4 = orc.e4m3_to_f32(np.arange(256, dtype=np.uint8)).astype(np.float64)
    e4 = np.unique(e4[np.isfinite(e4)])
    nearest = e4[np.abs(p8[:, None] - e4[None, :]).argmin(1)]
    assert (np.abs(p8 - nearest) <= 1e-5 * np.maximum(np.abs(nearest), 1e-3)).all()
    # the unrounded probabilities (relative to the same max) are mostly not E4M3 values
    p = np.exp2((s - m) * float(np.float32(CL_HANDMADE)))
    near_p = e4[np.abs(p[:, None] - e4[None, :]).argmin(1)]
    assert (np.abs(p - near_p) > 1e-3 * p).mean() > 0.8


def test_block32_and_block64_decisions_differ():
    """With a rise of 5.25 log2 units in block 1 the 32-key decisions keep the stale max (p8 = E4M3(2^5.25) = 40)
    and the 64-key decision does not (key 0 gets E4M3(2^-5.25) = 13 * 2^-9): the normalised outputs differ, so a
    gate at block_n 32 distinguishes the two."""
    s = np.zeros(64, dtype=np.int64)
    s[0] = 8
    s[40] = 8 + 42                                     # 42 / 8 = 5.25 log2 units above key 0
    q8, qs, k8, ks, v8, vs = _handmade(s)
    o32 = orc.attention(q8, qs, k8, ks, v8, vs, 64, out_dtype="f32", block_n=32)
    o64 = orc.attention(q8, qs, k8, ks, v8, vs, 64, out_dtype="f32", block_n=64)
    p8, _ = _p8(s)
    assert abs(p8[40] - 40.0) < 1e-4
    assert not np.array_equal(o32, o64)
    assert abs(o32[0, 0, 0, 40] / o32[0, 0, 0, 0] - 40.0) < 1e-4
    assert abs(o64[0, 0, 0, 40] / o64[0, 0, 0, 0] - 512.0 / 13.0) < 1e-3


@pytest.mark.parametrize("causal", [False, True])
def test_attention_on_sampled_query_rows(causal):
    """q_rows / seq_q: the emulation of a subset of query rows equals those rows of the whole emulation bit for bit
    (causal offsets and split rows refer to the rows' positions)."""
    q, k, v = _bf16((1, 2, 200, 64), 60), _bf16((1, 2, 260, 64), 61), _bf16((1, 2, 260, 64), 62)
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v)
    rows_split = np.zeros((1, 2, 200), dtype=bool)
    rows_split[:, 1, 128:] = True
    full = orc.attention(q8, qs, k8, ks, v8, vs, 260, causal=causal, kv_split=(3, rows_split))
    sel = np.r_[0:10, 120:140, 190:200]
    part = orc.attention(np.ascontiguousarray(q8[:, :, sel]), np.ascontiguousarray(qs[:, :, sel]), k8, ks, v8, vs,
                         260, causal=causal, kv_split=(3, rows_split[:, :, sel]), q_rows=sel, seq_q=200)
    assert np.array_equal(part, full[:, :, sel])


def test_seed_binade_holds_the_scores_of_each_head_dim():
    """The seeded read F = c + S * 2^-26 is exact exactly while the int32 sum stays in c's binade: check the two
    ends by the int32 pattern arithmetic the kernel relies on, and which head dims the kernels seed."""
    c_bits = int(np.array([orc.SEED], dtype=np.float32).view(np.uint32)[0])
    assert c_bits == 0x3E22F983 and abs(orc.SEED - 1 / (2 * math.pi)) < 2.0 ** -26

    def read(s):  # the accumulator's int32 bits read as fp32
        return float(np.array([c_bits + s], dtype=np.int64).astype(np.uint32).view(np.float32)[0])

    # the ends: 1/8 and 1/4 themselves read right (mantissa 0); one step further the ulp changes
    for s in (-2292099, -1, 0, 1, 2064512, 6096509):
        assert Fraction(read(s)) == Fraction(orc.SEED) + Fraction(s, 2 ** 26), s
    for s in (-2292100, -4129024, 6096510):
        assert Fraction(read(s)) != Fraction(orc.SEED) + Fraction(s, 2 ** 26), s
    # |S| <= 127^2 * (channels one MFMA sum covers); d96 runs 96 nonzero channels of the 128 layout
    assert orc.seeded(64) and orc.seeded(96) and orc.seeded(128) and not orc.seeded(256)
    assert 127 * 127 * 128 <= 2292099 < 127 * 127 * 256
