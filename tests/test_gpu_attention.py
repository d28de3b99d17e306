"""gfx950 attention kernel vs the CPU emulation of the reference's quantized math and vs float attention.

Tolerances (north star): max |out - emulation| <= 2e-2 with the emulation taking the reference's lazy-rescale
decisions once per 32-key block (kernel_build/compile_attn.py:19), and cosine >= 0.999 against float attention; the
reference's own gate is cosine > 0.998 (tests/test_attention.py:54).  Beyond the north star, the kernel follows the
emulation element by element: the exp2 implementation and the fp32 summation order inside the PV MFMA are the only
differences, so most output elements are the emulation's bits and the rest move by a probability whose E4M3 rounding
flipped.  The test asserts >= 95% (bf16) / 85% (fp16) of the elements bit-identical and the largest difference within
1% of the largest |output|.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cdna4_sage
from cdna4_sage import _capi
from gpu_util import assert_near_walk, cosine, hnd_np, kv_split
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
COS = 0.999
SAME_BITS = {torch.bfloat16: 0.95, torch.float16: 0.85}  # fraction of output elements equal to the emulation's
MAX_REL = 1e-2                                           # max |out - emulation| / max |emulation|

CASES = [  # B, H, Hkv, Sq, Skv, D, dtype, layout, causal
    (1, 2, 2, 300, 300, 128, torch.bfloat16, "HND", False),
    (2, 4, 2, 515, 515, 64, torch.float16, "NHD", False),
    (1, 2, 2, 1000, 1000, 128, torch.bfloat16, "HND", True),
    (1, 4, 1, 257, 257, 64, torch.bfloat16, "HND", True),
    (1, 2, 2, 130, 777, 128, torch.float16, "HND", False),
    (1, 3, 3, 1024, 64, 128, torch.bfloat16, "NHD", False),
    (3, 2, 2, 77, 1031, 128, torch.bfloat16, "HND", False),
    (1, 8, 8, 1024, 1024, 64, torch.bfloat16, "HND", False),   # config 1 shape
    (1, 2, 2, 130, 777, 128, torch.float16, "HND", True),      # bottom-right causal, q_len < kv_len
    (2, 4, 2, 300, 1000, 64, torch.bfloat16, "NHD", True),
    (1, 2, 2, 300, 300, 96, torch.bfloat16, "HND", False),     # head_dim 96: no rotation, 128-channel layout
    (1, 4, 2, 257, 600, 96, torch.float16, "NHD", True),
    (1, 2, 2, 300, 500, 256, torch.bfloat16, "HND", False),    # head_dim 256: block-diagonal rotation
    (2, 2, 1, 200, 200, 256, torch.float16, "NHD", True),
    (1, 8, 8, 1024, 1024, 256, torch.bfloat16, "HND", False),  # several split key ranges
    # one to three key tiles: the prologue loads the first tile and prefetches the second when there is one
    (1, 2, 2, 96, 33, 128, torch.bfloat16, "HND", False),      # one partial tile
    (1, 2, 2, 200, 100, 64, torch.float16, "HND", False),      # a whole tile and a partial one
    (1, 2, 2, 128, 128, 128, torch.bfloat16, "NHD", True),     # two whole tiles, causal
    (2, 2, 1, 70, 190, 128, torch.bfloat16, "HND", True),      # three tiles, causal with q_len < kv_len
    # wider GQA groups and a larger batch: 8 query heads per kv head (causal), multi-query (16 per kv head), batch 4
    (2, 32, 4, 700, 700, 128, torch.bfloat16, "HND", True),
    (1, 16, 1, 300, 900, 64, torch.float16, "NHD", False),
    (4, 8, 2, 257, 513, 128, torch.bfloat16, "NHD", True),
]


def _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    return q, k, v


def _emulate(q, k, v, layout, causal, sm_scale=None, out_dtype="bf16", split=None, walk=False):
    """Emulation with the reference's 32-key rescale blocks, following the kernel's split plan (`split`, from
    gpu_util.kv_split).  walk=True also returns the reference's one walk over every key (no split), or None when
    nothing is split."""
    qn, kn, vn = hnd_np(q, layout), hnd_np(k, layout), hnd_np(v, layout)
    q8, qs = orc.quant_q(qn, sm_scale)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(kn.shape[2]))
    emu = orc.attention(q8, qs, k8, ks, v8, vs, kn.shape[2], causal=causal, block_n=32, out_dtype=out_dtype,
                        kv_split=split, also_unsplit=walk and split is not None)
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal, sm_scale=sm_scale)
    if walk:
        emu, wk = emu if split is not None else (emu, None)
        return emu, ref, wk
    return emu, ref


@pytest.mark.parametrize("B,H,Hkv,Sq,Skv,D,dt,layout,causal", CASES)
def test_attention_vs_emulation(dev, B, H, Hkv, Sq, Skv, D, dt, layout, causal):
    q, k, v = _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=Sq + Skv)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), tensor_layout=layout, is_causal=causal)
    assert out.shape == q.shape and out.dtype == dt
    got = hnd_np(out, layout)
    split = kv_split(dev, B, H, Sq, Skv, D, causal)
    emu, ref, walk = _emulate(q, k, v, layout, causal, out_dtype="bf16" if dt == torch.bfloat16 else "f16",
                              split=split, walk=True)
    err = float(np.abs(got - emu).max())
    c = cosine(got, ref)
    assert err <= MAX_ABS, err
    assert c >= COS, c
    same = float((got == emu).mean())
    assert same >= SAME_BITS[dt], same
    assert err <= MAX_REL * float(np.abs(emu).max()), (err, float(np.abs(emu).max()))
    if walk is not None:   # split tiles, also against the reference's one walk over every key
        assert_near_walk(got, walk, ref)


@pytest.mark.parametrize("D,dt,causal", [(128, torch.bfloat16, False), (64, torch.float16, True),
                                         (96, torch.bfloat16, False), (256, torch.float16, False)])
def test_degenerate_inputs_vs_emulation(dev, D, dt, causal):
    """Inputs that reach the quantizers' clamps, through the whole forward: zero query rows (scale 1e-12 / 127, every
    score of the row 0, so uniform weights over the visible keys), a zero 32-key K block (scale 1e-12 / 127, those
    scores 0), a head whose keys are all equal (uniform weights on every row), a zero V channel (VS = 0: that output
    channel is exactly 0) and a constant V channel (every E4M3 code 448).  Against the emulation and float64
    attention with the gates above."""
    B, H, Hkv, Sq, Skv = 1, 2, 2, 300, 333
    g = torch.Generator().manual_seed(31 + D)
    q = torch.randn(B, H, Sq, D, generator=g)
    k = torch.randn(B, Hkv, Skv, D, generator=g)
    v = torch.randn(B, Hkv, Skv, D, generator=g)
    q[:, :, 10] = 0.0
    q[:, 1, 200:260] = 0.0
    k[:, 0, 64:96] = 0.0
    k[:, 1] = k[:, 1, :1].clone()
    v[..., 9] = 0.0
    v[..., 17] = 0.75
    q, k, v = (t.to(dt) for t in (q, k, v))
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), is_causal=causal)
    got = hnd_np(out)
    assert np.isfinite(got).all()
    assert (got[..., 9] == 0).all()
    split = kv_split(dev, B, H, Sq, Skv, D, causal)
    emu, ref, walk = _emulate(q, k, v, "HND", causal, out_dtype="bf16" if dt == torch.bfloat16 else "f16",
                              split=split, walk=True)
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS, err
    assert cosine(got, ref) >= COS
    assert float((got == emu).mean()) >= SAME_BITS[dt]
    if walk is not None:
        assert_near_walk(got, walk, ref)


def test_sm_scale(dev):
    q, k, v = _inputs(1, 2, 2, 600, 600, 128, torch.bfloat16, "HND", seed=7)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND", sm_scale=0.05)
    emu, ref = _emulate(q, k, v, "HND", False, sm_scale=0.05, split=kv_split(dev, 1, 2, 600, 600, 128, False))
    got = hnd_np(out)
    assert float(np.abs(got - emu).max()) <= MAX_ABS
    assert cosine(got, ref) >= COS


def test_flux_config2_full(dev):
    """Config 2 (Flux 1x24x4608x128 bf16, outlier K channels): cosine vs fp32 attention on all heads, and the
    emulation on a two-head sample (the per-head computation is independent of the other heads).  Heads 21 and 22
    hold the tiles of the short last round, which the kernel's plan splits on a 256-CU device: the sample covers
    whole and split tiles."""
    from cdna4_sage.configs import CONFIGS, make_inputs

    cfg = CONFIGS["2"]
    q, k, v = make_inputs(cfg)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), "HND")
    ref = F.scaled_dot_product_attention(q.to(dev).float(), k.to(dev).float(), v.to(dev).float())
    c = F.cosine_similarity(out.float().flatten(), ref.flatten(), dim=0).item()
    assert c >= COS, c
    qs_, ks_, vs_ = make_inputs(cfg, heads=slice(21, 23))
    split = kv_split(dev, cfg.B, cfg.H, cfg.S, cfg.S, cfg.D, False, heads=[21, 22])
    emu, ref2, walk = _emulate(qs_, ks_, vs_, "HND", False, split=split, walk=True)
    got = out[:, 21:23].float().cpu().numpy()
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS, err
    assert float((got == emu).mean()) >= SAME_BITS[torch.bfloat16]
    assert err <= MAX_REL * float(np.abs(emu).max())
    if walk is not None:
        # the split rows (heads 21-22 hold 60 of the 96 split tiles) against the reference's one walk over every
        # key: measured max 4.9e-4 on the emulation, 90% of their elements bit-identical
        rows = split[1]
        gap = assert_near_walk(got, walk, ref2)
        assert gap <= 2e-3, gap
        assert float((got[rows] == walk[rows]).mean()) >= 0.85


@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 2, 600, 600, 128), (2, 4, 515, 515, 64), (3, 2, 77, 1031, 128)])
def test_split_plan_and_unsplit_call(dev, B, H, Sq, Skv, D):
    """Small problems fill one partial round, so the plan splits their key range; a call without workspace runs
    every tile whole and must match the unsplit emulation, the default call the split one."""
    n_full, chunks, ws = _capi.attn_plan(dev.index or 0, B, H, Sq, Skv, D, False)
    n_split = B * H * ((Sq + 127) // 128)
    # per row of each chunk: fp16 O / l (D values) and fp32 (m, l)
    assert n_full == 0 and chunks >= 2 and ws == n_split * chunks * 128 * (2 * D + 8)
    q, k, v = _inputs(B, H, H, Sq, Skv, D, torch.bfloat16, "HND", seed=B + Sq)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    from gpu_util import run_quant_kv, run_quant_q
    q8, qs = (torch.from_numpy(a).to(dev) for a in run_quant_q(qd))
    k8, ks, v8t, vs = (torch.from_numpy(a).to(dev) for a in run_quant_kv(kd, vd))
    st = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for wsz in (0, ws):
        out = torch.empty(B, H, Sq, D, device=dev, dtype=torch.bfloat16)
        buf = torch.empty(max(wsz, 1), device=dev, dtype=torch.uint8)
        _capi.call("sage_attn_fwd", q8.data_ptr(), qs.data_ptr(), k8.data_ptr(), ks.data_ptr(), v8t.data_ptr(),
                   vs.data_ptr(), out.data_ptr(), out.stride(0), out.stride(2), out.stride(1), B, H, H, Sq, Skv, D,
                   0, _capi.DTYPE_BF16, None, buf.data_ptr() if wsz else None, wsz, st)
        outs.append(out.float().cpu().numpy())
    with pytest.raises(_capi.SageError, match="workspace"):
        _capi.call("sage_attn_fwd", q8.data_ptr(), qs.data_ptr(), k8.data_ptr(), ks.data_ptr(), v8t.data_ptr(),
                   vs.data_ptr(), out.data_ptr(), out.stride(0), out.stride(2), out.stride(1), B, H, H, Sq, Skv, D,
                   0, _capi.DTYPE_BF16, None, buf.data_ptr(), ws - 1, st)
    whole, _ = _emulate(q, k, v, "HND", False)
    split, ref = _emulate(q, k, v, "HND", False, split=(chunks, np.ones((B, H, Sq), dtype=bool)))
    assert float(np.abs(outs[0] - whole).max()) <= MAX_ABS
    assert float(np.abs(outs[1] - split).max()) <= MAX_ABS
    assert cosine(outs[1], ref) >= COS
    assert_near_walk(outs[1], whole, ref)   # the split call against the reference's one walk over every key


def test_split_range_whose_probabilities_underflow(dev):
    """Key 0 leads every other key by 124-152 in the exponent: the later ranges of the split (plan: one tile, 4
    ranges), started from the max after key tile 0, hold l in (0, 2^-128) on most rows and O = 0.  The kernel must
    store their partials as 0 (no 0 * inf = NaN from 1 / l) and give the emulation's output, V of key 0."""
    from gpu_util import underflow_split_inputs

    q, k, v = underflow_split_inputs()
    split = kv_split(dev, 1, 1, 128, 1024, 128, False)
    assert split is not None and split[0] >= 2
    qt, kt, vt = (torch.from_numpy(a).to(torch.bfloat16) for a in (q, k, v))
    out = cdna4_sage.attention(qt.to(dev), kt.to(dev), vt.to(dev), "HND")
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    q8, qs = orc.quant_q(q)
    k8, ks, v8, vs = orc.quant_kv(k, v, seq_pad=_capi.kv_pad(1024))
    emu, walk = orc.attention(q8, qs, k8, ks, v8, vs, 1024, block_n=32, kv_split=split, also_unsplit=True)
    assert float(np.abs(got - emu).max()) <= MAX_ABS
    assert_near_walk(got, walk, orc.sdpa_reference(q, k, v))


def test_split_merge_is_deterministic_across_calls(dev):
    """Split tiles are merged from partials in a workspace that every call reuses.  Repeated calls that alternate
    two inputs must reproduce each output bit for bit: a merge that read stale partials of the previous call, or
    depended on the order in which chunks finished, would not."""
    from cdna4_sage.configs import CONFIGS, make_inputs

    cfg = CONFIGS["2"]
    a = [t.to(dev) for t in make_inputs(cfg)]
    b = [t.flip(2).contiguous() for t in a]
    outs = [cdna4_sage.attention(*(a if i % 2 == 0 else b), "HND").clone() for i in range(6)]
    torch.cuda.synchronize()
    for i in range(2, 6):
        assert torch.equal(outs[i], outs[i % 2]), i
    assert not torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("D", [80, 512])
def test_unsupported_head_dims(dev, D):
    q = torch.randn(1, 2, 256, D, device=dev, dtype=torch.bfloat16)
    with pytest.raises(cdna4_sage.Unsupported):
        cdna4_sage.attention(q, q, q, "HND")
