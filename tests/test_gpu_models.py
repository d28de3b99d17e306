"""The reference's model-benchmark shapes (tests/bench_models.py:15-42, cdna4_sage.configs.MODEL_SHAPES: SD / SDXL /
SD3.5, Flux, Qwen-Image, HiDream, Neta Lumina, Anima, Wan, HunyuanVideo, LTXV, CogVideoX, AuraFlow and three causal
shapes; self- and cross-attention, HND and NHD, bf16 and fp16, head dims 40 to 256) through the kernel-forced call at
their full size, each checked against the oracle on sampled heads:

* the quantizers' Q8 / QS / K8 / KS / V8T / VS of the head bit-exact;
* the attention output against the emulation (the reference's 32-key rescale decisions, the kernel's split plan) on
  the first, middle and last query tiles and the split tiles of the head, max-abs <= 2e-2, with the share of
  bit-equal elements of the other GPU gates (95% bf16, 85% fp16); split rows also against the reference's one walk
  over every key;
* cosine >= 0.999 against float32 attention over the whole head.

Head dim 40 is not a kernel shape: the call raises Unsupported, and the router sends it to SDPA as the reference does.
Inputs are N(0, 1) as in the reference's benchmark, drawn on the GPU from a seeded generator."""
import numpy as np
import pytest
import torch

import cdna4_sage
from cdna4_sage import _capi
from cdna4_sage.configs import MODEL_SHAPES
from gpu_util import assert_near_walk, fp32_cos_head, kv_split, run_quant_kv, run_quant_q, unpad
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
COS = 0.999
BM = 128  # query rows per attention workgroup
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}
SAME_BITS = {"bf16": 0.95, "f16": 0.85}


def _tiles(Sq, H, b, h, n_full):
    """First, middle and last query tile of head (b, h), and the tail round's first split tile and the whole tile
    before it when they fall in this head."""
    q_tiles = (Sq + BM - 1) // BM
    pick = {0, q_tiles // 2, q_tiles - 1}
    first_split = n_full - (b * H + h) * q_tiles
    if 0 < first_split < q_tiles:
        pick |= {first_split - 1, first_split}
    return np.concatenate([np.arange(t * BM, min(Sq, (t + 1) * BM)) for t in sorted(pick)])


@pytest.mark.parametrize("idx", range(len(MODEL_SHAPES)), ids=[s[0] for s in MODEL_SHAPES])
def test_model_shape_vs_oracle(dev, idx):
    name, B, Sq, Skv, H, D, layout, dtn, causal = MODEL_SHAPES[idx]
    dt = DTYPES[dtn]
    g = torch.Generator(device=dev)
    g.manual_seed(7000 + idx)
    shape = (lambda s: (B, H, s, D)) if layout == "HND" else (lambda s: (B, s, H, D))  # noqa: E731
    q, k, v = (torch.randn(shape(s), generator=g, device=dev, dtype=torch.float32).to(dt) for s in (Sq, Skv, Skv))
    if D not in cdna4_sage.HEAD_DIMS:
        with pytest.raises(cdna4_sage.Unsupported):
            cdna4_sage.attention(q, k, v, tensor_layout=layout, is_causal=causal)
        return
    out = cdna4_sage.attention(q, k, v, tensor_layout=layout, is_causal=causal)
    assert out.shape == q.shape and out.dtype == dt
    hnd = (lambda t: t) if layout == "HND" else (lambda t: t.transpose(1, 2))  # noqa: E731
    qh, kh, vh, oh = hnd(q), hnd(k), hnd(v), hnd(out)
    n_full, _, _ = _capi.attn_plan(dev.index or 0, B, H, Sq, Skv, D, causal)
    skp = _capi.kv_pad(Skv)
    for b, h in sorted({(0, 0), (B - 1, H - 1)}):
        q1, k1, v1 = (t[b:b + 1, h:h + 1].contiguous() for t in (qh, kh, vh))
        qn, kn, vn = (t.float().cpu().numpy() for t in (q1, k1, v1))
        # quantizers of this head, bit-exact
        q8, qs = orc.quant_q(qn)
        k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=skp)
        g_q8, g_qs = run_quant_q(q1)
        g_k8, g_ks, g_v8t, g_vs = run_quant_kv(k1, v1)
        assert np.array_equal(unpad(g_q8, D), q8) and np.array_equal(g_qs.view(np.uint32), qs.view(np.uint32))
        assert np.array_equal(unpad(g_k8, D), k8) and np.array_equal(g_ks.view(np.uint32), ks.view(np.uint32))
        assert np.array_equal(unpad(g_vs, D).view(np.uint32), vs.view(np.uint32))
        assert np.array_equal(unpad(g_v8t, D, axis=2), orc.v8_to_device_layout(v8))
        # attention on sampled query tiles against the emulation over every key
        rows = _tiles(Sq, H, b, h, n_full)
        split = kv_split(dev, B, H, Sq, Skv, D, causal, heads=[h])
        if split is not None:
            split = (split[0], split[1][b:b + 1][:, :, rows])
        emu = orc.attention(np.ascontiguousarray(q8[:, :, rows]), np.ascontiguousarray(qs[:, :, rows]), k8, ks, v8, vs,
                            Skv, causal=causal, block_n=32, out_dtype=dtn, kv_split=split, q_rows=rows, seq_q=Sq,
                            also_unsplit=split is not None)
        emu, walk = emu if split is not None else (emu, None)
        got = oh[b, h][torch.from_numpy(rows).to(dev)].float().cpu().numpy()
        err = float(np.abs(got - emu[0, 0]).max())
        same = float((got == emu[0, 0]).mean())
        print(f"{name} b={b} h={h}: {len(rows)} rows, max |out - emu| = {err:.3g}, bit-equal {same:.4f}", flush=True)
        assert err <= MAX_ABS, (name, b, h, err)
        assert same >= SAME_BITS[dtn], (name, b, h, same)
        if walk is not None and split[1].any():
            sel = split[1][0, 0]
            ref = orc.sdpa_reference(qn[:, :, rows[sel]], kn, vn)[0, 0]
            assert_near_walk(got[sel], walk[0, 0][sel], ref)
        # cosine against float32 attention over the whole head
        cos = fp32_cos_head(qh[b, h].float(), kh[b, h].float(), vh[b, h].float(), oh[b, h], causal)
        assert cos >= COS, (name, b, h, cos)
