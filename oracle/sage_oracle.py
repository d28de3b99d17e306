"""CPU restatement of the reference's quantized SageAttention math (numpy, float32 / float64).

TEST INFRASTRUCTURE ONLY.  This module is the checker for the gfx950 HIP path: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``cdna4_sage``) never calls it and fails loudly when the HIP library is missing.

What each function restates (paths relative to the reference checkout):

* ``hadamard_pm1``      src/rdna4_sage/_attention.py:48-56 (Sylvester +-1 matrix, order RB = head_dim for
                        head_dim 64 / 128, kernel_build/build_kernels.py:40-41, :102-104).
* ``fwht_rows``         the rotation x = row @ Hm of kernel_build/sage_quant.py:12-30 (`_load_qk`).  The
                        reference accumulates the +-1 products in fp32 inside ``tl.dot`` in an order that the
                        gfx12 hardware fixes and that is not recoverable here.  This build defines the rotation
                        as a float64 fast Walsh-Hadamard transform in a fixed stage order (stage bit 0 first,
                        then 1, 2, ...; butterfly (a, b) -> (a + b, a - b)), rounded once to float32.  For bf16
                        and fp16 rows every float64 partial sum is exact unless a row spans more than ~2^38 in
                        magnitude, so the result is the correctly rounded fp32 of the exact sum; it equals the
                        reference's fp32 accumulation whenever that accumulation is exact.  The HIP kernels run
                        the same stages in the same order, so the two agree bit for bit in every case.
* ``quant_q``           kernel_build/sage_quant.py:33-48 (`_quant_q`) plus the sm_scale fold of
                        src/rdna4_sage/_attention.py:130-131.
* ``v_amax``            src/rdna4_sage/_attention.py:120-121 (`vector_norm(v, inf, dim=seq, dtype=fp32)`).
* ``quant_kv``          kernel_build/sage_quant.py:51-70 (`_quant_kv`).
* ``f32_to_e4m3``       the fp32 -> float8 E4M3FN cast of sage_quant.py:70 (round to nearest even, subnormals
                        kept; inputs are clamped to +-448 first so the NaN code is never produced).
* ``attention``         the FlyDSL kernel's math as rewritten by kernel_build/make_sage.py:75-107, :196-237,
                        make_sage_r2.py:54-269 and make_sage_pkg.py:74-87: int32 S = Q8 K8^T, per-32-key K scale,
                        lazy rescale with threshold 8.0 (log2 units), exp2, P cast to E4M3, fp32 PV
                        accumulation, epilogue (O * ((1/448) / l)) * VS.  ``block_n`` is the key block of the
                        online softmax, one lazy-rescale decision each: 32 in the reference
                        (kernel_build/compile_attn.py:19); the gfx950 kernel walks 64-key tiles but decides per
                        32-key block as well, so the GPU tests compare at 32 (64 serves the oracle's own
                        identities).  Split key ranges and additive-mask classes follow the kernel's 64-key tiles
                        whatever block_n.  For head dims up to 128 the exponent argument is the gfx950 kernel's
                        fma(c + S * 2^-26, ct * 2^26, nk) form (c = fp32(1 / (2 pi))), which differs from the
                        reference's S * ct - cl * m by the rounding of nk (at most 1.5 * ct: S moved by less than
                        2 units, far below the int8 quantization error of S and the E4M3 step of p); head dim 256
                        uses fma(fp32(S), ct, -cl * m), the reference's own form, and so do 32-row groups whose
                        scales are large enough for the seeded form's rounding to matter (``wide_rows``: the
                        kernel's own rule, pinned by the single-key bound at scale 100 in tests/test_oracle.py).
                        Bottom-right causal for any q_len / kv_len: query i sees keys j <= i + kv_len - q_len; a
                        query that sees no key (q_len > kv_len) gives a 0 row (the gfx950 convention; the reference
                        sends such calls to SDPA, so this case has no reference value).
                        ``attn_mask`` (bool, True = attend, broadcastable to [B, H, Sq, Skv]) masks scores to
                        -inf like the causal mask.  The reference sends every masked call to torch SDPA
                        (src/rdna4_sage/__init__.py:78-79); the quantized masked math here is this build's own
                        definition, pinned by the all-True, causal-equivalent and padding-equivalent identities
                        in tests/test_oracle.py and by the float64 masked softmax ``sdpa_reference``.  A float
                        ``attn_mask`` is additive (SDPA's convention); the kernel's bias path (``_bias_tile``) is
                        pinned by the all-zero (= no mask), {0, -inf} (= the boolean mask) and per-row-constant
                        (softmax shift invariance) identities and by float64 attention with the same bias.
* ``sage_forward_varlen`` src/sageattention/core.py:66-89 (`sageattn_varlen`): one ``sage_forward`` per sequence
                        of the packed batch.
* ``lse_reference``     src/sageattention/core.py:23-44 (`_lse`).

All float32 steps are written as float32 numpy operations, which round to nearest even like the GPU's
float32 ALU.  ``exp2`` and the order of the fp32 additions inside the PV product are implementation-defined
on both sides; the attention output is therefore compared with a tolerance, while Q8 / K8 / V8 and their
scales are compared bit for bit.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
KV_BLOCK = 32          # one K scale per 32 keys (kernel_build/build_kernels.py:30)
E4M3_MAX = 448.0
RESCALE_THRESHOLD = 8.0  # make_sage.py:219-225: keep a stale max until it is exceeded by 2^8
LOG2E = 1.4426950408889634  # the reference's _LOG2E (python float)
# fp32(1 / (2 pi)) = 0x3E22F983, the gfx950 kernel's seed of the QK accumulators for head dims up to 128: the int32
# sum read as fp32 is c + S * 2^-26 exactly for -2,292,099 <= S <= 6,096,509 (see seeded()), so it needs no conversion
SEED = float(np.array([0x3E22F983], dtype=np.uint32).view(np.float32)[0])
SEED_ULP = 2.0 ** -26
# Large scales: a 32-row group (a wave) whose largest K scale over the keys exceeds fp32(CT_WIDE / its largest
# cl * 2^26) reads its scores exactly (F - c) with the offset -(cl * m), the reference's form; the seeded form's
# rounding of c * ct grows with ct
CT_WIDE = 2.0 ** 18
# the gfx950 kernel's key tile: split key ranges and the classes of additive masks are per 64-key tile, whatever the
# block_n of the online softmax
KERNEL_TILE = 64


def seeded(d_layout: int) -> bool:
    """Whether the gfx950 kernel reads its scores seeded (F = c + S * 2^-26) for a layout of d_layout channels:
    c + S * 2^-26 is exact (inside c's binade [1/8, 1/4], whose ends read right) for -2,292,099 <= S <= 6,096,509,
    i.e. |S| <= 127^2 * d_layout for d_layout <= 128.  Head dim 256 (|S| up to 4,129,024) converts S to fp32
    instead (F = S), the reference's arithmetic."""
    return 127 * 127 * d_layout < 2292099


# ----------------------------------------------------------------------------------------------------------
# bf16 / fp16 helpers (inputs are kept as float32 arrays holding exactly representable bf16 / fp16 values)
# ----------------------------------------------------------------------------------------------------------
def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value (RNE), returned as float32."""
    b = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    nan = np.isnan(x)
    out = rounded.astype(np.uint32).view(F32).copy()
    out[nan] = np.nan
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(F32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (round_to_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


# ----------------------------------------------------------------------------------------------------------
# Hadamard rotation
# ----------------------------------------------------------------------------------------------------------
def hadamard_pm1(d: int) -> np.ndarray:
    """Sylvester +-1 matrix of order d (src/rdna4_sage/_attention.py:48-56): H1 = [1], H2n = [[H, H], [H, -H]]."""
    h = np.ones((1, 1), dtype=np.float64)
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    return h


def fwht_rows(x: np.ndarray) -> np.ndarray:
    """Rotate the last axis by the unnormalised Sylvester Hadamard matrix (x @ H, H symmetric).

    float64 butterflies, stage bit 0 first; returns float64 (round with ``.astype(np.float32)``)."""
    x = np.array(x, dtype=np.float64, copy=True)
    d = x.shape[-1]
    assert d & (d - 1) == 0, "power-of-two head_dim only"
    lead = x.shape[:-1]
    s = 1
    while s < d:
        v = x.reshape(*lead, d // (2 * s), 2, s)
        a = v[..., 0, :].copy()
        b = v[..., 1, :]
        v[..., 0, :] = a + b
        v[..., 1, :] = a - b
        s *= 2
    return x


def rotation_block(d: int) -> int:
    """Channels of one Hadamard block for head_dim d: min(d, 128) for powers of two (kernel_build/build_kernels.py:27,
    HADAMARD_MAX = 128; rotates() :40-41 applied at :102-104: block-diagonal for d = 256, sage_quant.py:18-30), 0 (no
    rotation) otherwise (d = 96)."""
    return min(d, 128) if d & (d - 1) == 0 else 0


def rotate_rows(x: np.ndarray) -> np.ndarray:
    """The quantizers' rotation of the last axis (float64): one Sylvester Hadamard per block of rotation_block(d)
    channels, or a plain float64 copy when d is not rotated."""
    d = x.shape[-1]
    rb = rotation_block(d)
    if rb == 0:
        return np.array(x, dtype=np.float64, copy=True)
    lead = x.shape[:-1]
    return fwht_rows(np.asarray(x).reshape(*lead, d // rb, rb)).reshape(*lead, d)


# ----------------------------------------------------------------------------------------------------------
# Rounding helpers
# ----------------------------------------------------------------------------------------------------------
def round_half_away_i8(y: np.ndarray) -> np.ndarray:
    """int8(trunc(y >= 0 ? fp32(y + 0.5) : fp32(y - 0.5)))  (sage_quant.py:44, :65)."""
    y = y.astype(F32)
    t = np.where(y >= 0, y + F32(0.5), y - F32(0.5)).astype(F32)
    return np.trunc(t).astype(np.int8)


def f32_to_e4m3(y: np.ndarray) -> np.ndarray:
    """float32 -> OCP float8 E4M3FN bits (uint8), round to nearest even, subnormals kept.

    Inputs must already lie in [-448, 448] (the quantizer clamps); NaN is never produced."""
    y = np.ascontiguousarray(y, dtype=F32)
    bits = y.view(np.uint32)
    sign = ((bits >> 31) & 1).astype(np.uint32) << 7
    a = np.abs(y)
    out = np.zeros(y.shape, dtype=np.uint32)
    normal = a >= F32(2.0 ** -6)
    # normal range: round the 23-bit mantissa to 3 bits (RNE) and rebias the exponent (127 -> 7)
    ab = a.view(np.uint32).astype(np.uint64)
    r = (ab + 0x7FFFF + ((ab >> 20) & 1)) >> 20
    nrm = (r - ((127 - 7) << 3)).astype(np.uint32)
    # subnormal range: value = m * 2^-9, m = RNE(a * 512) in 0..8 (8 is the smallest normal, code 0x08)
    sub = np.rint(a * F32(512.0)).astype(np.uint32)
    out = np.where(normal, nrm, sub)
    return (out | sign).astype(np.uint8)


def e4m3_to_f32(bits: np.ndarray) -> np.ndarray:
    """OCP E4M3FN bits -> float32 (0x7F / 0xFF decode to NaN)."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int32)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(F32)


# ----------------------------------------------------------------------------------------------------------
# Quantizers
# ----------------------------------------------------------------------------------------------------------
def qs_fold_factor(sm_scale, d: int):
    """None for the default scale, else fp32(sm_scale * sqrt(D)) (src/rdna4_sage/_attention.py:130-131).  A scale
    that is not positive (NaN included) is the default too: the reference's op passes `sm_scale if sm_scale > 0 else
    None` (src/rdna4_sage/ops.py:10)."""
    if sm_scale is None or not sm_scale > 0 or math.isclose(sm_scale, d ** -0.5, rel_tol=1e-6):
        return None
    return F32(sm_scale * math.sqrt(d))


def quant_q(q: np.ndarray, sm_scale=None):
    """q: [B, H, S, D] float32 holding bf16/fp16 values (HND).

    Returns (q8 int8 [B, H, S, D], qs float32 [B, H, S]).  sage_quant.py:33-48; scale / RB because the
    unnormalised Hadamard multiplies Q K^T by RB (:259-260), the scale itself without rotation (d = 96); optional
    sm_scale fold (_attention.py:130-131)."""
    d = q.shape[-1]
    rb = rotation_block(d)
    x = rotate_rows(q).astype(F32)
    a = np.maximum(np.abs(x).max(axis=-1), F32(1e-12)).astype(F32)
    s = (a / F32(127.0)).astype(F32)
    y = (x / s[..., None]).astype(F32)
    q8 = round_half_away_i8(y)
    qs = (s / F32(rb)).astype(F32) if rb else s
    f = qs_fold_factor(sm_scale, d)
    if f is not None:
        qs = (qs * f).astype(F32)
    return q8, qs


def v_amax(v: np.ndarray) -> np.ndarray:
    """v: [B, Hkv, S, D] -> per-channel max |v| over the sequence, float32 [B, Hkv, D] (_attention.py:120-121)."""
    if v.shape[2] == 0:
        return np.zeros(v.shape[:2] + v.shape[3:], dtype=F32)
    return np.abs(v.astype(F32)).max(axis=2).astype(F32)


def padded_len(s: int, multiple: int = 64) -> int:
    return (s + multiple - 1) // multiple * multiple


def quant_kv(k: np.ndarray, v: np.ndarray, vs: np.ndarray | None = None, seq_pad: int | None = None):
    """k, v: [B, Hkv, S, D] float32 holding bf16/fp16 values.

    Returns (k8 int8 [B, Hkv, Sp, D], ks float32 [B, Hkv, Sp/32], v8 uint8 E4M3 bits [B, Hkv, Sp, D],
    vs float32 [B, Hkv, D]) in natural key order; rows >= S are zero.  sage_quant.py:51-70."""
    B, Hkv, S, D = k.shape
    sp = padded_len(S, KV_BLOCK) if seq_pad is None else seq_pad
    assert sp % KV_BLOCK == 0 and sp >= S
    if vs is None:
        vs = v_amax(v)
    kp = np.zeros((B, Hkv, sp, D), dtype=F32)
    kp[:, :, :S] = k
    x = rotate_rows(kp).astype(F32).reshape(B, Hkv, sp // KV_BLOCK, KV_BLOCK, D)
    a = np.maximum(np.abs(x).max(axis=(-1, -2)), F32(1e-12)).astype(F32)
    ks = (a / F32(127.0)).astype(F32)
    y = (x / ks[..., None, None]).astype(F32)
    k8 = round_half_away_i8(y).reshape(B, Hkv, sp, D)
    vsc = np.maximum(vs.astype(F32), F32(1e-30))
    c = (F32(448.0) / vsc).astype(F32)
    vp = np.zeros((B, Hkv, sp, D), dtype=F32)
    vp[:, :, :S] = v
    yv = np.clip((vp * c[:, :, None, :]).astype(F32), F32(-448.0), F32(448.0))
    v8 = f32_to_e4m3(yv)
    return k8, ks, v8, vs.astype(F32)


# ----------------------------------------------------------------------------------------------------------
# Attention (tile-faithful float32 emulation)
# ----------------------------------------------------------------------------------------------------------
def logit_scale_base(d: int) -> np.float32:
    """fp32(sm_scale * LOG2E) with the kernel's built-in sm_scale = 1/sqrt(D) (make_sage.py:40-46, :76-80)."""
    return F32((1.0 / math.sqrt(d)) * LOG2E)


def attention(q8, qs, k8, ks, v8, vs, seq_kv: int, causal: bool = False, block_n: int = 32,
              out_dtype: str = "bf16", threshold: float = RESCALE_THRESHOLD, return_stats: bool = False,
              kv_split=None, attn_mask=None, q_rows=None, seq_q=None, also_unsplit=False):
    """Quantized attention as the reference kernel computes it.

    q8 [B, H, Sq, D] int8, qs [B, H, Sq] f32, k8 [B, Hkv, Sp, D] int8, ks [B, Hkv, Sp/32] f32,
    v8 [B, Hkv, Sp, D] E4M3 bits (natural key order), vs [B, Hkv, D] f32.  Returns float32 [B, H, Sq, D]
    holding values rounded to ``out_dtype`` ("bf16", "f16" or "f32" for no rounding).

    ``kv_split = (chunks, rows)``, rows a bool array [B, H, Sq], emulates the gfx950 kernel's split tiles (no
    counterpart in the reference): for those rows the keys run as ``chunks`` contiguous ranges (range c = the
    kernel's 64-key tiles [c * n // chunks, (c + 1) * n // chunks), n = ceil(seq_kv / 64), whatever ``block_n``),
    each with its own online softmax, l = 0, O = 0 and m = -inf, except that a range starting after the first 64-key
    kernel tile that any row of its 128-row block sees starts from the running max that the one-walk softmax has
    after that tile (the kernel's seed; without a mask that is tile 0), stored as
    (m_c, l_c, fp16(O_c / l_c)) and merged with M = max m_c, W_c = exp2((m_c - M) * cl) * l_c, L = sum W_c,
    O = sum W_c * fp16(O_c / l_c) (float32, chunk order), then the usual epilogue with L.  A range in which a row
    sees no key (l_c = 0, m_c = -inf) stores 0 and weighs 0.

    ``attn_mask``: bool array broadcastable to [B, H, Sq, seq_kv], True where the query attends the key (the
    convention of torch SDPA's boolean masks; no counterpart in the reference's kernel, which sends masked calls to
    SDPA).  Masked scores are -inf like the causal ones, ANDed with the causal mask when both are given.  A float
    array is an additive mask (SDPA: softmax(Q K^T * scale + mask), -inf = masked), emulated as the gfx950 kernel
    runs it: per 32-row group (a wave) and key tile whose values are all 0 or -inf, the boolean path above; otherwise
    the bias path of ``_online_softmax``.  The group-and-tile classes are per 32 rows and 64 keys (the kernel's tile),
    whatever ``block_n``.

    ``q_rows`` (int array, with ``seq_q``): the query axis of q8 / qs holds only these rows of a query sequence of
    length seq_q (a sample of a long problem; the bottom-right causal mask and ``kv_split`` rows refer to these
    positions).  Not combined with ``attn_mask``.

    ``also_unsplit``: return ``(out, out_unsplit)``, where ``out_unsplit`` walks every key of the split rows in one
    online softmax, as the reference does (kernel_build/make_sage_r2.py:141-253); it is computed on the way."""
    B, H, Sq, D = q8.shape
    Hkv = k8.shape[1]
    assert block_n % KV_BLOCK == 0 and KERNEL_TILE % block_n == 0 and H % Hkv == 0
    grp = H // Hkv
    hk = np.arange(H) // grp
    cl = (logit_scale_base(D) * qs.astype(F32)).astype(F32)      # [B, H, Sq]
    n_tiles = (seq_kv + block_n - 1) // block_n
    # split key ranges are whole kernel tiles: range c = kernel tiles [c * n // chunks, (c + 1) * n // chunks)
    k_tiles = (seq_kv + KERNEL_TILE - 1) // KERNEL_TILE
    per = KERNEL_TILE // block_n
    def krange(c, chunks):
        return min(c * k_tiles // chunks * per, n_tiles), min((c + 1) * k_tiles // chunks * per, n_tiles)
    if attn_mask is not None:
        attn_mask = np.asarray(attn_mask)
        if attn_mask.dtype == bool:
            attn_mask = np.broadcast_to(attn_mask, (B, H, q8.shape[2], seq_kv))
        else:
            attn_mask = np.broadcast_to(attn_mask.astype(F32), (B, H, q8.shape[2], seq_kv))
    if q_rows is not None:
        assert attn_mask is None and seq_q is not None and len(q_rows) == q8.shape[2]
        qpos = (np.asarray(q_rows, dtype=np.int64), int(seq_q))
    else:
        qpos = (np.arange(q8.shape[2]), q8.shape[2])
    wide = wide_rows(cl, ks, seq_kv, qpos[0], hk) if seeded(D) else None
    o, m, l = _online_softmax(q8, cl, k8, ks, v8, seq_kv, causal, block_n, threshold, 0, n_tiles, attn_mask, qpos,
                              wide)

    def epilogue(o, l):
        with np.errstate(divide="ignore"):
            inv = np.where(l > 0, (F32(1.0 / 448.0) / l).astype(F32), F32(0.0)).astype(F32)   # no visible key: 0
        res = ((o * inv[..., None]).astype(F32) * vs[:, hk][:, :, None, :].astype(F32)).astype(F32)
        return round_output(res, out_dtype)

    unsplit = epilogue(o, l) if also_unsplit else None
    if kv_split is not None:
        chunks, rows = kv_split
        # the kernel's seed: a range that starts after the first kernel tile its 128-row block visits starts from the
        # walk's running max after that tile, instead of from -inf (no mask: tile 0; the kernel splits only
        # non-causal calls without a mask, and masked calls with the causal flag folded into the mask)
        first, m_seed = _seed_tiles(q8, cl, k8, ks, v8, seq_kv, causal, block_n, threshold, attn_mask, qpos, wide)
        parts = []
        for c in range(chunks):
            lo = c * k_tiles // chunks
            m_init = None if first is None else np.where(lo > first, m_seed, F32(-np.inf)).astype(F32)
            parts.append(_online_softmax(q8, cl, k8, ks, v8, seq_kv, causal, block_n, threshold, *krange(c, chunks),
                                         attn_mask, qpos, wide, m_init=m_init))
        mm = parts[0][1]
        for _, mc, _ in parts[1:]:
            mm = np.maximum(mm, mc)
        ll = np.zeros_like(l)
        oo = np.zeros_like(o)
        for oc, mc, lc in parts:
            # each chunk's O is stored normalised by its own l, in fp16 (round to nearest even); a chunk without
            # a visible key (l = 0) stores 0 and weighs 0
            # (below 2^-64, l and O are scaled by 2^64 first, exactly, so that the reciprocal stays finite: a range
            # started from the seeded max can hold only probabilities far below it)
            with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
                ls = np.where(lc < F32(2.0 ** -64), F32(2.0 ** 64), F32(1.0)).astype(F32)
                rl = np.where(lc > 0, (F32(1.0) / (lc * ls).astype(F32)).astype(F32), F32(0.0)).astype(F32)
                pn = ((oc * ls[..., None]).astype(F32) * rl[..., None]).astype(F32).astype(np.float16).astype(F32)
                w = np.where(lc > 0, (np.exp2(((mc - mm).astype(F32) * cl).astype(F32)).astype(F32) * lc).astype(F32),
                             F32(0.0)).astype(F32)
            ll = (ll + w).astype(F32)
            oo = (oo + (w[..., None] * pn).astype(F32)).astype(F32)
        o = np.where(rows[..., None], oo, o)
        m = np.where(rows, mm, m)
        l = np.where(rows, ll, l)
    out = epilogue(o, l)
    if also_unsplit:
        assert not return_stats
        return out, unsplit
    if return_stats:
        return out, m, l
    return out


def _seed_tiles(q8, cl, k8, ks, v8, seq_kv, causal, block_n, threshold, attn_mask, qpos, wide):
    """Per row: the first 64-key kernel tile that any row of its 128-row block sees (int [B, H, Sq]; a block that
    sees no key gets a tile past the last), and the walk's running max after that tile.  (None, None) for a causal
    call without a mask, which the kernel never splits."""
    B, H, Sq = cl.shape
    n_tiles = (seq_kv + block_n - 1) // block_n
    per = KERNEL_TILE // block_n
    k_tiles = (seq_kv + KERNEL_TILE - 1) // KERNEL_TILE
    if attn_mask is None:
        if causal:
            return None, None
        first = np.zeros((B, H, Sq), dtype=np.int64)
    else:
        rows, seq_q = qpos
        vis = attn_mask if attn_mask.dtype == bool else attn_mask != -np.inf        # [B, H, Sq, seq_kv]
        if causal:
            vis = vis & (np.arange(seq_kv)[None, :] <= rows[:, None] + (seq_kv - seq_q))
        tile_vis = np.zeros((B, H, Sq, k_tiles), dtype=bool)
        for t in range(k_tiles):
            tile_vis[..., t] = vis[..., t * KERNEL_TILE:(t + 1) * KERNEL_TILE].any(axis=-1)
        blk = np.asarray(rows) // 128
        first = np.full((B, H, Sq), k_tiles, dtype=np.int64)
        for bb in np.unique(blk):
            sel = blk == bb
            any_t = tile_vis[:, :, sel].any(axis=2)                                   # [B, H, k_tiles]
            f = np.where(any_t.any(-1), any_t.argmax(-1), k_tiles)
            first[:, :, sel] = f[..., None]
    m_seed = np.full((B, H, Sq), -np.inf, dtype=F32)
    for f in np.unique(first):
        if f >= k_tiles:
            continue
        m_f = _online_softmax(q8, cl, k8, ks, v8, seq_kv, causal, block_n, threshold, 0, min((f + 1) * per, n_tiles),
                              attn_mask, qpos, wide)[1]
        m_seed = np.where(first == f, m_f, m_seed).astype(F32)
    return first, m_seed


def wide_rows(cl, ks, seq_kv, pos, hk):
    """Bool [B, H, Sq]: rows whose 32-row group (query positions pos // 32; with a sample of rows, the sampled rows
    of the group) reads its scores in the reference's form: the largest K scale of its kv head over the blocks of
    keys [0, seq_kv) exceeds fp32(CT_WIDE / the group's largest cl * 2^26).  cl [B, H, Sq], ks [B, Hkv, Sp/32]."""
    cls = (cl * F32(2.0 ** 26)).astype(F32)
    kmx = ks[:, :, :(seq_kv + KV_BLOCK - 1) // KV_BLOCK].astype(F32).max(axis=-1)[:, hk]      # [B, H]
    grp = np.asarray(pos) // 32
    out = np.zeros(cls.shape, dtype=bool)
    for g in np.unique(grp):
        sel = grp == g
        thr = (F32(CT_WIDE) / cls[..., sel].max(axis=-1)).astype(F32)                      # [B, H]
        out[..., sel] = (kmx > thr)[..., None]
    return out


def _online_softmax(q8, cl, k8, ks, v8, seq_kv, causal, block_n, threshold, t_lo, t_hi, attn_mask=None,
                    qpos=None, wide=None, m_init=None):
    """Online softmax over key tiles [t_lo, t_hi): unnormalised O, running max m and sum l per row.  attn_mask:
    None, bool [B, H, Sq, seq_kv] (True = attend) or float32 [B, H, Sq, seq_kv] (additive, -inf = masked).  qpos:
    (the rows' positions in the query sequence, its length), default all Sq rows.

    Bias path (float masks, tiles of a 32-row group holding a value other than 0 and -inf), in log2 units:
    t = fma(F, ct', fma(b, log2e, -fp32(c * ct'))) per score (F = c + S * 2^-26, ct' = ct * 2^26, c the seed; for
    head dim 256 F = S, ct' = ct, c = 0), the tile's row max of t against m * cl for the lazy rescale
    (m_new = m_cand * fp32(1 / cl) when it moves), p = exp2(t - cl * m_ref)."""
    B, H, Sq, D = q8.shape
    Hkv, Sp = k8.shape[1], k8.shape[2]
    hk = np.arange(H) // (H // Hkv)
    q8f = q8.astype(F32)
    k8f = k8.astype(F32)
    v8f = e4m3_to_f32(v8)
    m = np.full((B, H, Sq), -np.inf, dtype=F32) if m_init is None else np.array(m_init, dtype=F32)
    l = np.zeros((B, H, Sq), dtype=F32)
    o = np.zeros((B, H, Sq, D), dtype=F32)
    rows, seq_q = qpos if qpos is not None else (np.arange(Sq), Sq)   # query positions, query length
    causal_off = seq_kv - seq_q
    nsub = block_n // KV_BLOCK
    for t in range(t_lo, t_hi):
        j0 = t * block_n
        j1 = min(j0 + block_n, Sp)
        cols = np.arange(j0, j0 + block_n)
        kt = np.zeros((B, Hkv, block_n, D), dtype=F32)
        kt[:, :, : j1 - j0] = k8f[:, :, j0:j1]
        vt = np.zeros((B, Hkv, block_n, D), dtype=F32)
        vt[:, :, : j1 - j0] = v8f[:, :, j0:j1]
        # exact int32 scores (|S| <= 127 * 127 * 256 < 2^24, so every float32 partial sum is exact)
        s = np.matmul(q8f, np.swapaxes(kt[:, hk], -1, -2))      # [B, H, Sq, block_n]
        mask = cols[None, :] >= seq_kv
        if causal:
            mask = mask | (cols[None, :] > rows[:, None] + causal_off)
        bias_rows = None
        if attn_mask is not None:
            nv = max(0, min(j0 + block_n, seq_kv) - j0)
            if attn_mask.dtype == bool:
                am = np.zeros((B, H, Sq, block_n), dtype=bool)
                am[..., :nv] = attn_mask[..., j0:j0 + nv]
                mask = mask | ~am
            else:
                bt = np.full((B, H, Sq, block_n), -np.inf, dtype=F32)
                bt[..., :nv] = attn_mask[..., j0:j0 + nv]
                bt = np.where(mask, F32(-np.inf), bt).astype(F32)
                bias_rows = _bias_groups(attn_mask, seq_kv, causal, causal_off, j0 // KERNEL_TILE)
                mask = mask | (bt == -np.inf)
        s = np.where(mask, F32(-np.inf), s).astype(F32)
        kst = np.ones((B, Hkv, nsub), dtype=F32)
        nb = min(nsub, ks.shape[2] - j0 // KV_BLOCK)
        kst[:, :, :nb] = ks[:, :, j0 // KV_BLOCK: j0 // KV_BLOCK + nb]
        kst = kst[:, hk]                                          # [B, H, nsub]
        sb = s.reshape(B, H, Sq, nsub, KV_BLOCK)
        rowmax = (sb.max(axis=-1) * kst[:, :, None, :]).astype(F32).max(axis=-1)   # [B, H, Sq]
        m_cand = np.maximum(m, rowmax)
        with np.errstate(invalid="ignore"):
            need = ((m_cand - m).astype(F32) * cl).astype(F32) > F32(threshold)
        m_new = np.where(need, m_cand, m).astype(F32)
        # a row that has seen no key yet (causal with q_len > kv_len) keeps m = -inf and p = 0; the gfx950 kernel
        # offsets such rows from 0 instead of -inf so that corr and the exponents stay free of NaN (no counterpart
        # in the reference, which sends these calls to SDPA)
        m_ref = np.where(m_new == -np.inf, F32(0.0), m_new).astype(F32)
        with np.errstate(invalid="ignore"):
            corr = np.exp2(((m - m_ref).astype(F32) * cl).astype(F32)).astype(F32)
        neg = (F32(0.0) - (cl * m_ref).astype(F32)).astype(F32)
        ct = (cl[..., None] * kst[:, :, None, :]).astype(F32)    # [B, H, Sq, nsub]
        if seeded(D):
            # the gfx950 kernel reads S as F = c + S * 2^-26 (exact, c the seed) and folds the offset into the
            # additive term: arg = fma(F, ct', nk), ct' = ct * 2^26 (exact), nk = neg - fp32(c * ct').  F * ct' + nk
            # is exact in float64 (both terms have the magnitude of c * ct' and at most 48 significant bits), so
            # rounding it once to float32 is the kernel's fma.  It equals S * ct + neg up to the two roundings of
            # nk (each at most half an ulp of ~c * 2^26 * ct: <= 1.5 ct together).
            ct = (ct * F32(2.0 ** 26)).astype(F32)
            nk = (neg[..., None] - (F32(SEED) * ct).astype(F32)).astype(F32)
            fs = (sb * F32(SEED_ULP) + F32(SEED)).astype(F32)
            # rows of a wide group: F - c = S * 2^-26 (exact) and the offset without the seed term
            wb = np.broadcast_to(wide[..., None], ct.shape)                     # [B, H, Sq, nsub]
            nk = np.where(wb, neg[..., None], nk).astype(F32)
            fs = np.where(wb[..., None], (sb * F32(SEED_ULP)).astype(F32), fs).astype(F32)
            seed_t = np.where(wb, F32(0.0), F32(SEED)).astype(F32)
        else:
            # head dim 256: F = fp32(S), arg = fma(S, ct, neg), the reference's exponent (make_sage_r2.py:193-200).
            # S * ct is exact in float64; the sum is rounded twice (float64, then float32), which differs from the
            # fma's single rounding only when the float64 result lands on a float32 rounding boundary.
            nk = np.broadcast_to(neg[..., None], ct.shape).astype(F32)
            fs = sb.astype(F32)
            seed_t = F32(0.0)
        arg = (fs.astype(np.float64) * ct[..., None].astype(np.float64) + nk[..., None].astype(np.float64)).astype(F32)
        p = np.exp2(arg).astype(F32).reshape(B, H, Sq, block_n)
        if bias_rows is not None and bias_rows.any():
            p, corr, need, m_new = _bias_tile(fs, ct, bt, m, cl, threshold, bias_rows, p, corr, need, m_new, seed_t)
        tile_sum = p.sum(axis=-1, dtype=F32)
        l = ((corr * l).astype(F32) + tile_sum).astype(F32)
        o = np.where(need[..., None], (o * corr[..., None]).astype(F32), o)
        p8 = e4m3_to_f32(f32_to_e4m3(p))
        o = (o + np.matmul(p8, vt[:, hk])).astype(F32)
        m = m_new
    return o, m, l


def _bias_tile(fs, ct, bt, m, cl, threshold, rows, p, corr, need, m_new, seed=SEED):
    """The bias path of one tile for the rows in `rows` (other rows keep p, corr, need, m_new as given).  fs: the
    scores as the kernel reads them [B, H, Sq, nsub, 32]; ct [B, H, Sq, nsub] (scaled by 2^26 like the kernel's
    when seeded); bt: the additive mask of the tile [B, H, Sq, block_n]; seed: c, or 0 for unseeded scores and wide
    blocks (a scalar or [B, H, Sq, nsub])."""
    B, H, Sq = m.shape
    nsub = ct.shape[-1]
    f64 = np.float64
    bb = bt.reshape(B, H, Sq, nsub, KV_BLOCK)
    nseed = -(F32(seed) * ct).astype(F32)                                 # -fp32(c * ct'), -0 unseeded
    with np.errstate(invalid="ignore", over="ignore"):
        inner = (bb.astype(f64) * f64(F32(LOG2E)) + nseed[..., None].astype(f64)).astype(F32)
        t = (fs.astype(f64) * ct[..., None].astype(f64) + inner.astype(f64)).astype(F32)
    t = t.reshape(B, H, Sq, -1)
    rowmax = t.max(axis=-1)
    with np.errstate(invalid="ignore"):
        mc = (m * cl).astype(F32)
        mcand = np.maximum(mc, rowmax).astype(F32)
        nd = (mcand - mc).astype(F32) > F32(threshold)
    rcl = (F32(1.0) / cl).astype(F32)
    mn = np.where(nd, (mcand * rcl).astype(F32), m).astype(F32)
    mref = np.where(mn == -np.inf, F32(0.0), mn).astype(F32)
    with np.errstate(invalid="ignore"):
        cr = np.exp2(((m - mref).astype(F32) * cl).astype(F32)).astype(F32)
    negl = (F32(0.0) - (cl * mref).astype(F32)).astype(F32)
    pb = np.exp2((t + negl[..., None]).astype(F32)).astype(F32)
    return (np.where(rows[..., None], pb, p), np.where(rows, cr, corr), np.where(rows, nd, need),
            np.where(rows, mn, m_new).astype(F32))


def _bias_groups(attn_mask, seq_kv, causal, causal_off, kt):
    """Bool [B, H, Sq]: rows whose 32-row group (a wave of the gfx950 kernel) takes the bias path in kernel tile kt
    (keys [64 kt, 64 kt + 64)): some value of the group's rows over the tile's keys, after the padding and causal
    masks, is neither 0 nor -inf."""
    B, H, Sq, _ = attn_mask.shape
    j0 = kt * KERNEL_TILE
    nv = max(0, min(j0 + KERNEL_TILE, seq_kv) - j0)
    bt = np.full((B, H, Sq, KERNEL_TILE), -np.inf, dtype=F32)
    bt[..., :nv] = attn_mask[..., j0:j0 + nv]
    if causal:
        cols = np.arange(j0, j0 + KERNEL_TILE)
        bt = np.where(cols[None, :] > np.arange(Sq)[:, None] + causal_off, F32(-np.inf), bt).astype(F32)
    general = (bt != 0) & (bt != -np.inf)
    ng = (Sq + 31) // 32
    grp = np.zeros((B, H, ng), dtype=bool)
    for g in range(ng):
        grp[:, :, g] = general[:, :, 32 * g:32 * g + 32].any(axis=(-1, -2))
    return grp[:, :, np.arange(Sq) // 32]


def split_rows(B: int, H_total: int, Sq: int, n_full: int, heads=None, block_m: int = 128) -> np.ndarray:
    """Bool [B, len(heads), Sq]: rows of the query tiles numbered >= n_full, where the gfx950 kernel numbers the
    tile of row r of batch b, head h as (b * H_total + h) * ceil(Sq / block_m) + r // block_m.  ``heads`` lists the
    heads of a sample by their index in the full problem (default: all H_total heads)."""
    heads = np.arange(H_total) if heads is None else np.asarray(heads)
    q_tiles = (Sq + block_m - 1) // block_m
    tile = ((np.arange(B)[:, None, None] * H_total + heads[None, :, None]) * q_tiles
            + (np.arange(Sq) // block_m)[None, None, :])
    return tile >= n_full


def round_output(x: np.ndarray, out_dtype: str) -> np.ndarray:
    if out_dtype == "bf16":
        return round_to_bf16(x)
    if out_dtype == "f16":
        return x.astype(np.float16).astype(F32)
    return x.astype(F32)


def sage_forward(q, k, v, causal=False, sm_scale=None, block_n=32, out_dtype="bf16", attn_mask=None, kv_split=None):
    """Full quantized path on HND float32 arrays holding bf16 / fp16 values: quant_q, quant_kv, attention."""
    q8, qs = quant_q(q, sm_scale)
    k8, ks, v8, vs = quant_kv(k, v)
    return attention(q8, qs, k8, ks, v8, vs, k.shape[2], causal=causal, block_n=block_n, out_dtype=out_dtype,
                     attn_mask=attn_mask, kv_split=kv_split)


def sage_forward_varlen(q, k, v, cu_q, cu_k, causal=False, sm_scale=None, block_n=32, out_dtype="bf16"):
    """Packed variable-length forward (src/sageattention/core.py:80-88: one call per sequence, NHD slices).
    q [total_q, H, D], k / v [total_k, Hkv, D] float32 arrays holding bf16 / fp16 values; cu_q / cu_k [batch + 1].
    Each sequence is quantized and attended on its own (sage_forward on its slices, bottom-right causal).  A sequence
    with queries but no keys gives 0 rows; rows outside every sequence are NaN (the gfx950 path leaves them
    unwritten)."""
    out = np.full(q.shape, np.nan, dtype=F32)
    for i in range(len(cu_q) - 1):
        q0, q1, k0, k1 = int(cu_q[i]), int(cu_q[i + 1]), int(cu_k[i]), int(cu_k[i + 1])
        if q1 == q0:
            continue
        if k1 == k0:
            out[q0:q1] = 0.0
            continue
        hnd = lambda t: np.ascontiguousarray(t.transpose(1, 0, 2))[None]   # noqa: E731  [1, H, S, D]
        o = sage_forward(hnd(q[q0:q1]), hnd(k[k0:k1]), hnd(v[k0:k1]), causal=causal, sm_scale=sm_scale,
                         block_n=block_n, out_dtype=out_dtype)
        out[q0:q1] = o[0].transpose(1, 0, 2)
    return out


# ----------------------------------------------------------------------------------------------------------
# Textbook references used to bound the emulation
# ----------------------------------------------------------------------------------------------------------
def sdpa_reference(q, k, v, causal=False, sm_scale=None, attn_mask=None):
    """float64 softmax attention, bottom-right causal, GQA by head repetition; attn_mask: bool (True = attend) or float
    (added to the scaled scores), broadcastable to [B, H, Sq, Skv].  A row that sees no key is 0."""
    B, H, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    rep = H // Hkv
    kk = np.repeat(k.astype(np.float64), rep, axis=1)
    vv = np.repeat(v.astype(np.float64), rep, axis=1)
    scale = D ** -0.5 if sm_scale is None else sm_scale
    s = np.matmul(q.astype(np.float64), np.swapaxes(kk, -1, -2)) * scale
    if causal:
        mask = np.arange(Skv)[None, :] > np.arange(Sq)[:, None] + (Skv - Sq)
        s = np.where(mask, -np.inf, s)
    if attn_mask is not None:
        am = np.asarray(attn_mask)
        if am.dtype == bool:
            s = np.where(np.broadcast_to(am, s.shape), s, -np.inf)
        else:
            s = s + np.broadcast_to(am.astype(np.float64), s.shape)
    mx = s.max(axis=-1, keepdims=True)
    seen = np.isfinite(mx)
    p = np.exp(s - np.where(seen, mx, 0.0))
    den = p.sum(axis=-1, keepdims=True)
    p = np.where(seen, p / np.where(seen, den, 1.0), 0.0)
    return np.matmul(p, vv)


def lse_reference(q, k, causal=False, sm_scale=None):
    """logsumexp_j(q_i . k_j * scale) in float64 (src/sageattention/core.py:23-44), [B, H, Sq]."""
    B, H, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    kk = np.repeat(k.astype(np.float64), H // Hkv, axis=1)
    scale = D ** -0.5 if sm_scale is None else sm_scale
    s = np.matmul(q.astype(np.float64), np.swapaxes(kk, -1, -2)) * scale
    if causal:
        mask = np.arange(Skv)[None, :] > np.arange(Sq)[:, None] + (Skv - Sq)
        s = np.where(mask, -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    return (np.log(np.exp(s - mx).sum(axis=-1)) + mx[..., 0])


# ----------------------------------------------------------------------------------------------------------
# Layout helpers shared with the tests (device layouts of the HIP path)
# ----------------------------------------------------------------------------------------------------------
def v8_to_device_layout(v8: np.ndarray) -> np.ndarray:
    """Natural [B, Hkv, Sp, D] E4M3 -> the HIP path's transposed V8T [B, Hkv, D, Sp].

    Within every 64-key group the keys are stored as the 4-key chunks of lane-half 0 first
    (keys 8g + 0..3, g = 0..7), then those of lane-half 1 (keys 8g + 4..7): key 8g + 4h + r sits at
    position 32h + 4g + r."""
    B, Hkv, Sp, D = v8.shape
    assert Sp % 64 == 0
    t = np.swapaxes(v8, -1, -2)                                  # [B, Hkv, D, Sp]
    t = t.reshape(B, Hkv, D, Sp // 64, 8, 2, 4)                  # key = 64G + 8g + 4h + r
    t = np.swapaxes(t, -3, -2)                                   # -> [.., G, h, g, r]
    return np.ascontiguousarray(t.reshape(B, Hkv, D, Sp))


def v8_from_device_layout(v8t: np.ndarray) -> np.ndarray:
    B, Hkv, D, Sp = v8t.shape
    t = v8t.reshape(B, Hkv, D, Sp // 64, 2, 8, 4)
    t = np.swapaxes(t, -3, -2).reshape(B, Hkv, D, Sp)
    return np.ascontiguousarray(np.swapaxes(t, -1, -2))
