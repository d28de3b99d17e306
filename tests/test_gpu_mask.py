"""attn_mask on the gfx950 kernel (sage_forward_masked: bool masks, and additive float masks of the inputs' dtype) vs
the CPU emulation with the same mask and vs the float64 masked softmax.

Tolerances as for the unmasked kernel: max |out - emulation| <= 2e-2 (emulation with the reference's 32-key
rescale blocks and the kernel's split plan) and cosine >= 0.999 against float attention with the mask.  Identities: an all-True mask gives the
unmasked kernel's output bit for bit; a mask whose rows see no key gives 0 rows and no NaN elsewhere.  The reference
sends masked calls to torch SDPA (src/rdna4_sage/__init__.py:78-79); its tests have no masked case.
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
# element-level agreement with the emulation, as for the unmasked kernel (tests/test_gpu_attention.py): measured
# 98.3-99.2% (bf16) / 93-96% (fp16) of the output elements bit-identical, largest difference 0.65% of max |output|
SAME_BITS = {torch.bfloat16: 0.95, torch.float16: 0.85}
MAX_REL = 1e-2
COS = 0.999


def _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    return q, k, v


def _emulate(q, k, v, layout, causal, mask, split, out_dtype):
    """Emulation with the mask following the kernel's split plan, float64 attention, and the reference's one walk
    over every key (None when the plan splits nothing)."""
    qn, kn, vn = hnd_np(q, layout), hnd_np(k, layout), hnd_np(v, layout)
    q8, qs = orc.quant_q(qn)
    k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(kn.shape[2]))
    m = mask.cpu().numpy() if mask.dtype == torch.bool else mask.float().cpu().numpy()
    emu = orc.attention(q8, qs, k8, ks, v8, vs, kn.shape[2], causal=causal, block_n=32, out_dtype=out_dtype,
                        kv_split=split, attn_mask=m, also_unsplit=split is not None)
    ref = orc.sdpa_reference(qn, kn, vn, causal=causal, attn_mask=m)
    emu, walk = emu if split is not None else (emu, None)
    return emu, ref, walk


def _key_padding(B, Skv, lengths):
    return torch.arange(Skv)[None, None, None, :] < torch.tensor(lengths)[:, None, None, None]


def _block_diagonal(S, bounds):
    seg = torch.zeros(S, dtype=torch.long)
    for b in bounds:
        seg[b:] += 1
    return (seg[:, None] == seg[None, :])[None, None]


def _random(shape, p, seed):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(shape, generator=g) < p
    return m


def _cases():
    c = []
    # B, H, Hkv, Sq, Skv, D, dtype, layout, causal, mask builder
    c.append(("key padding", (2, 2, 2, 300, 1031, 128, torch.bfloat16, "HND", False),
              lambda: _key_padding(2, 1031, [700, 1031])))
    c.append(("random full", (1, 2, 1, 257, 400, 64, torch.float16, "NHD", False),
              lambda: _random((1, 2, 257, 400), 0.7, 1)))
    c.append(("causal + key padding", (1, 2, 2, 500, 500, 128, torch.bfloat16, "HND", True),
              lambda: _key_padding(1, 500, [450])))
    c.append(("block diagonal", (1, 2, 2, 1000, 1000, 128, torch.bfloat16, "HND", False),
              lambda: _block_diagonal(1000, [130, 512, 700])))
    c.append(("2-D mask, GQA, d256", (2, 4, 2, 200, 333, 256, torch.bfloat16, "NHD", False),
              lambda: _random((200, 333), 0.5, 2)))
    c.append(("head_dim 96", (1, 2, 2, 300, 300, 96, torch.float16, "HND", False),
              lambda: _random((1, 1, 300, 300), 0.8, 3)))
    c.append(("causal q < kv, random", (1, 3, 3, 130, 777, 64, torch.bfloat16, "HND", True),
              lambda: _random((1, 3, 130, 777), 0.6, 4)))
    return c


CASES = _cases()


@pytest.mark.parametrize("name,shape,make_mask", CASES, ids=[c[0] for c in CASES])
def test_masked_attention_vs_emulation(dev, name, shape, make_mask):
    B, H, Hkv, Sq, Skv, D, dt, layout, causal = shape
    q, k, v = _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=Sq + Skv + D)
    mask = make_mask()
    if name == "random full":
        mask[0, 1, 7] = False           # a row that sees no key
        mask[0, 0, 9] = False
        mask[0, 0, 9, 399] = True       # a row that sees one key of the last (partial) tile
    print(f"case {name}: B={B} H={H} Hkv={Hkv} Sq={Sq} Skv={Skv} D={D} {dt} {layout} causal={causal} "
          f"mask {tuple(mask.shape)}", flush=True)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), tensor_layout=layout, is_causal=causal,
                               attn_mask=mask.to(dev))
    assert out.shape == q.shape and out.dtype == dt
    got = hnd_np(out, layout)
    assert np.isfinite(got).all()
    split = kv_split(dev, B, H, Sq, Skv, D, False)   # the masked call uses the dense non-causal plan
    full = torch.broadcast_to(mask, (B, H, Sq, Skv))
    emu, ref, walk = _emulate(q, k, v, layout, causal, full, split, "bf16" if dt == torch.bfloat16 else "f16")
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS, err
    assert cosine(got, ref) >= COS
    assert float((got == emu).mean()) >= SAME_BITS[dt]
    assert err <= MAX_REL * float(np.abs(emu).max())
    if walk is not None:   # split tiles, also against the reference's one walk over every key
        assert_near_walk(got, walk, ref)
    if name == "random full":
        assert (got[0, 1, 7] == 0).all() and (ref[0, 1, 7] == 0).all()
        assert np.abs(got[0, 0, 9] - emu[0, 0, 9]).max() <= MAX_ABS


def test_all_true_mask_is_the_unmasked_kernel(dev):
    """Every tile of an all-True mask takes the mask-free body, the partial last tile the bit-masked one: the output
    must equal the unmasked call bit for bit (same plan, same arithmetic)."""
    q, k, v = (t.to(dev) for t in _inputs(1, 4, 2, 700, 1100, 128, torch.bfloat16, "HND", seed=5))
    base = cdna4_sage.attention(q, k, v)
    for m in (torch.ones(1100, dtype=torch.bool), torch.ones(1, 4, 700, 1100, dtype=torch.bool)):
        assert torch.equal(cdna4_sage.attention(q, k, v, attn_mask=m.to(dev)), base)


def test_flux_size_identities(dev):
    """Config 2 (Flux 1x24x4608x128) at full size, by size-independent properties: an all-True mask is the unmasked
    call bit for bit (whole and split tiles of the plan), and a key-padding mask that hides the last 512 keys equals
    the call whose padding mask is the kv_len bound, i.e. every output row differs from the unmasked call and none is
    NaN; a mask hiding everything gives zeros."""
    from cdna4_sage.configs import CONFIGS, make_inputs
    cfg = CONFIGS["2"]
    q, k, v = (t.to(dev) for t in make_inputs(cfg))
    base = cdna4_sage.attention(q, k, v)
    S = cfg.S
    assert torch.equal(cdna4_sage.attention(q, k, v, attn_mask=torch.ones(S, dtype=torch.bool, device=dev)), base)
    pad = torch.arange(S, device=dev) < S - 512
    out = cdna4_sage.attention(q, k, v, attn_mask=pad)
    assert torch.isfinite(out).all() and not torch.equal(out, base)
    ref = F.scaled_dot_product_attention(q[:, :2].float(), k[:, :2].float(), v[:, :2].float(), attn_mask=pad)
    assert cosine(out[:, :2].float().cpu().numpy(), ref.cpu().numpy()) >= COS
    none = cdna4_sage.attention(q, k, v, attn_mask=torch.zeros(S, dtype=torch.bool, device=dev))
    assert (none == 0).all()


@pytest.mark.parametrize("kind", ["bool", "float"])
def test_flux_size_key_masks_vs_emulation(dev, kind):
    """Config 2 (Flux 1x24x4608x128) at full size with bench.py's key-padding mask (the first 4032 of 4608 keys
    visible) or an additive per-key bias of the inputs' dtype (+-2 on those keys, -inf on the rest), against the
    emulation with the same mask on sampled query tiles of two heads: the first, middle and last tile and the split
    tiles of the plan; split rows also against the one walk, and float32 masked attention over the whole head."""
    from cdna4_sage.configs import CONFIGS, make_inputs
    cfg = CONFIGS["2"]
    S, D = cfg.S, cfg.D
    q, k, v = make_inputs(cfg)
    vis = torch.arange(S) < S - S // 8
    if kind == "bool":
        mask = vis
    else:
        g = torch.Generator().manual_seed(12)
        mask = torch.where(vis, torch.rand(S, generator=g) * 4 - 2, torch.tensor(float("-inf"))).to(cfg.dtype)
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    out = cdna4_sage.attention(qd, kd, vd, attn_mask=md)
    assert torch.isfinite(out).all()
    n_full, _, _ = _capi.attn_plan(dev.index or 0, cfg.B, cfg.H, S, S, D, False)
    m = mask.numpy() if kind == "bool" else mask.float().numpy()
    q_tiles = S // 128
    for h in (0, cfg.H - 1):
        pick = {0, q_tiles // 2, q_tiles - 1}
        first_split = n_full - h * q_tiles
        if 0 < first_split < q_tiles:
            pick |= {first_split - 1, first_split}
        rows = np.concatenate([np.arange(t * 128, (t + 1) * 128) for t in sorted(pick)])
        qn, kn, vn = (t[:, h:h + 1].float().numpy() for t in (q, k, v))
        q8, qs = orc.quant_q(qn)
        k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=_capi.kv_pad(S))
        split = kv_split(dev, cfg.B, cfg.H, S, S, D, False, heads=[h])
        if split is not None:
            split = (split[0], split[1][:, :, rows])
        # the mask does not depend on the query row, so whole sampled tiles stand for a query sequence of their own
        emu = orc.attention(np.ascontiguousarray(q8[:, :, rows]), np.ascontiguousarray(qs[:, :, rows]), k8, ks, v8, vs,
                            S, block_n=32, kv_split=split, attn_mask=m[None, None, None, :],
                            also_unsplit=split is not None)
        emu, walk = emu if split is not None else (emu, None)
        got = out[0, h][torch.from_numpy(rows).to(dev)].float().cpu().numpy()
        err = float(np.abs(got - emu[0, 0]).max())
        same = float((got == emu[0, 0]).mean())
        print(f"flux {kind} mask head {h}: {len(rows)} rows, max |out - emu| = {err:.3g}, bit-equal {same:.4f}",
              flush=True)
        assert err <= MAX_ABS and same >= SAME_BITS[cfg.dtype], (h, err, same)
        if walk is not None and split[1].any():
            sel = split[1][0, 0]
            ref = orc.sdpa_reference(qn[:, :, rows[sel]], kn, vn, attn_mask=m[None, None, None, :])[0, 0]
            assert_near_walk(got[sel], walk[0, 0][sel], ref)
        fm = md if kind == "bool" else md.float()
        ref32 = F.scaled_dot_product_attention(qd[:, h:h + 1].float(), kd[:, h:h + 1].float(), vd[:, h:h + 1].float(),
                                               attn_mask=fm)
        assert cosine(out[:, h:h + 1].float().cpu().numpy(), ref32.cpu().numpy()) >= COS


def test_fully_masked_rows_and_tiles_give_zero(dev):
    q, k, v = (t.to(dev) for t in _inputs(2, 2, 2, 300, 600, 64, torch.float16, "HND", seed=6))
    none = torch.zeros(2, 1, 1, 600, dtype=torch.bool, device=dev)
    out = cdna4_sage.attention(q, k, v, attn_mask=none)
    assert torch.isfinite(out).all() and (out == 0).all()
    half = torch.ones(2, 2, 300, 600, dtype=torch.bool, device=dev)
    half[1, :, 128:] = False        # whole query tiles (split or not) without any visible key
    out = cdna4_sage.attention(q, k, v, attn_mask=half)
    assert (out[1, :, 128:] == 0).all() and torch.equal(out[0], cdna4_sage.attention(q, k, v)[0])


def test_sageattn_routes_bool_masks_to_the_kernel(dev, monkeypatch):
    """sageattn (and sageattention.sageattn through kwargs) runs boolean masks, and additive ones of the inputs'
    dtype, on the kernel above the routing threshold; CDNA4_SAGE_NATIVE_MASK=0 restores the reference's SDPA
    routing."""
    import sageattention
    monkeypatch.setattr(cdna4_sage, "MIN_WORK", 0)      # 8 x 1024 x 1024 is below the default threshold
    q, k, v = (t.to(dev) for t in _inputs(1, 8, 8, 1024, 1024, 64, torch.bfloat16, "HND", seed=7))
    mask = _key_padding(1, 1024, [900]).to(dev)
    kern = cdna4_sage.attention(q, k, v, attn_mask=mask)
    assert torch.equal(cdna4_sage.sageattn(q, k, v, attn_mask=mask), kern)
    assert torch.equal(sageattention.sageattn(q, k, v, attn_mask=mask), kern)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=mask)
    assert cosine(kern.float().cpu().numpy(), ref.cpu().numpy()) >= COS
    fmask = torch.zeros(1, 1, 1, 1024, device=dev, dtype=torch.bfloat16)
    fmask[..., 900:] = float("-inf")
    assert torch.equal(cdna4_sage.sageattn(q, k, v, attn_mask=fmask), kern)   # the same mask as an additive one
    # a query row that sees no key: 0 on the kernel route, and 0 from torch SDPA (this torch, bool mask, bf16) on
    # the reference's routing; every other row is the same on both routes as above
    rowmask = torch.ones(1, 1, 1024, 1024, dtype=torch.bool, device=dev)
    rowmask[..., 7, :] = False
    kern_rows = cdna4_sage.sageattn(q, k, v, attn_mask=rowmask)
    assert (kern_rows[:, :, 7] == 0).all() and torch.isfinite(kern_rows).all()
    monkeypatch.setattr(cdna4_sage, "NATIVE_MASK", False)
    assert torch.equal(cdna4_sage.sageattn(q, k, v, attn_mask=mask), cdna4_sage._torch_sdpa(q, k, v, attn_mask=mask))
    sdpa_rows = cdna4_sage.sageattn(q, k, v, attn_mask=rowmask)
    ref_rows = cdna4_sage._torch_sdpa(q, k, v, attn_mask=rowmask)
    assert torch.equal(sdpa_rows.isnan(), ref_rows.isnan())
    assert torch.equal(torch.nan_to_num(sdpa_rows), torch.nan_to_num(ref_rows))
    assert torch.equal(sdpa_rows[:, :, 7], kern_rows[:, :, 7])     # both routes: 0


def _alibi(H, Sq, Skv, slope=0.03):
    rel = (torch.arange(Sq)[:, None] + (Skv - Sq) - torch.arange(Skv)[None, :]).abs().float()
    return -(slope * torch.arange(1, H + 1).float())[:, None, None] * rel[None]    # [H, Sq, Skv]


FLOAT_CASES = [
    # name, (B, H, Hkv, Sq, Skv, D, dtype, layout, causal), mask builder (float32, cast to the inputs' dtype)
    ("alibi", (1, 2, 2, 300, 700, 128, torch.bfloat16, "HND", False), lambda: _alibi(2, 300, 700)[None]),
    ("alibi causal fp16", (1, 2, 2, 257, 600, 128, torch.float16, "NHD", True), lambda: _alibi(2, 257, 600)[None]),
    ("padding as -inf + bias tiles", (2, 2, 1, 200, 1031, 64, torch.bfloat16, "HND", False), None),
    ("per-row bias, GQA d256", (1, 4, 2, 130, 333, 256, torch.bfloat16, "HND", False),
     lambda: torch.randn(1, 4, 130, 1) * 2.0),
]


@pytest.mark.parametrize("name,shape,make_mask", FLOAT_CASES, ids=[c[0] for c in FLOAT_CASES])
def test_float_mask_vs_emulation(dev, name, shape, make_mask):
    B, H, Hkv, Sq, Skv, D, dt, layout, causal = shape
    q, k, v = _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=Sq + Skv + 7)
    if make_mask is None:
        # zero tiles, -inf tiles (padding past 900 keys in batch 1), and tiles with a general bias (keys 128-255)
        mask = torch.zeros(B, 1, Sq, Skv)
        mask[1, :, :, 900:] = float("-inf")
        mask[:, :, :, 128:256] = torch.linspace(-3.0, 2.0, 128)
    else:
        mask = make_mask()
    mask = mask.to(dt)
    print(f"case {name}: B={B} H={H} Hkv={Hkv} Sq={Sq} Skv={Skv} D={D} {dt} {layout} causal={causal} "
          f"mask {tuple(mask.shape)}", flush=True)
    out = cdna4_sage.attention(q.to(dev), k.to(dev), v.to(dev), tensor_layout=layout, is_causal=causal,
                               attn_mask=mask.to(dev))
    got = hnd_np(out, layout)
    assert np.isfinite(got).all()
    split = kv_split(dev, B, H, Sq, Skv, D, False)
    full = torch.broadcast_to(mask, (B, H, Sq, Skv))
    emu, ref, walk = _emulate(q, k, v, layout, causal, full, split, "bf16" if dt == torch.bfloat16 else "f16")
    err = float(np.abs(got - emu).max())
    assert err <= MAX_ABS, err
    assert cosine(got, ref) >= COS
    assert float((got == emu).mean()) >= SAME_BITS[dt]
    assert err <= MAX_REL * float(np.abs(emu).max())
    if walk is not None:   # split tiles, also against the reference's one walk over every key
        assert_near_walk(got, walk, ref)


def test_float_mask_identities(dev):
    """An all-zero float mask is the unmasked kernel bit for bit (every tile mask-free); a float mask of 0 / -inf is
    the bool mask bit for bit (the same bit path); a bias constant along each row gives the unmasked output up to the
    rounding of the bias path (softmax is shift-invariant)."""
    q, k, v = (t.to(dev) for t in _inputs(1, 4, 2, 700, 1100, 128, torch.bfloat16, "HND", seed=11))
    base = cdna4_sage.attention(q, k, v)
    assert torch.equal(cdna4_sage.attention(q, k, v, attn_mask=torch.zeros(1100, dtype=torch.bfloat16, device=dev)),
                       base)
    boolm = _random((1, 4, 700, 1100), 0.7, 12).to(dev)
    fm = torch.zeros(boolm.shape, dtype=torch.bfloat16, device=dev).masked_fill(~boolm, float("-inf"))
    assert torch.equal(cdna4_sage.attention(q, k, v, attn_mask=fm), cdna4_sage.attention(q, k, v, attn_mask=boolm))
    shift = (torch.randn(1, 4, 700, 1, device=dev) * 5).to(torch.bfloat16)
    out = cdna4_sage.attention(q, k, v, attn_mask=shift)
    assert float((out.float() - base.float()).abs().max()) <= MAX_ABS
    assert cosine(out.float().cpu().numpy(), base.float().cpu().numpy()) >= 0.9999


def test_masked_op_and_graph_capture(dev):
    """torch.ops.cdna4_sage.attention_masked is the same call, and the masked forward (mask preparation, quantizers,
    attention, merge) replays under a HIP graph with the eager result on every replay."""
    q, k, v = (t.to(dev) for t in _inputs(1, 4, 4, 520, 520, 128, torch.bfloat16, "HND", seed=8))
    mask = _random((1, 1, 520, 520), 0.75, 9).to(dev)
    eager = cdna4_sage.attention(q, k, v, attn_mask=mask)
    op = torch.ops.cdna4_sage.attention_masked(q, k, v, mask, "HND", 0.0, False)
    assert torch.equal(op.transpose(1, 2), eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        cdna4_sage.attention(q, k, v, attn_mask=mask)           # warm-up: workspace sizes cached, allocator primed
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gout = cdna4_sage.attention(q, k, v, attn_mask=mask)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, eager), i
        cdna4_sage.attention(q, k, v)                              # eager work between replays
        torch.cuda.synchronize()
