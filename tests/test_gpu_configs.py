"""BASELINE configurations 3, 4, 5a and 5b on their real workloads (cdna4_sage.configs.make_inputs: Wan 2.1 14B
[1, 40, 32760, 128] with x10 outlier channels, HunyuanVideo [1, 24, 67320, 128] with a shared K bias, causal GQA
[2, 32/8, 8192, 128] and [2, 16/4, 8192, 64] with return_lse), through the public sageattention.sageattn call.

Per configuration, on sampled heads at the full sequence length:
* the quantizers' Q8 / QS / K8 / KS / V8T / VS bit-exact against the oracle;
* the attention output against the emulation (the reference's 32-key rescale decisions, the kernel's split plan) on
  sampled query tiles (first, middle, last, and whole and split tiles of the tail round), max-abs <= 2e-2;
* cosine >= 0.999 against float32 attention over whole sampled heads;
* with return_lse, the LSE of sampled rows against the float64 logsumexp at the reference's atol 2e-3 / rtol 1e-4
  (tests/test_sageattention.py:70).
"""
import numpy as np
import pytest
import torch

import sageattention
from cdna4_sage import _capi
from cdna4_sage.configs import CONFIGS, make_inputs
from gpu_util import assert_near_walk, fp32_cos_head, kv_split, run_quant_kv, run_quant_q
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
COS = 0.999
BM = 128  # query rows per attention workgroup


def _tiles(cfg, n_full, head_flat):
    """Query tiles to emulate for head head_flat (b * H + h): first, middle, last, and the tail round's first split
    tile and the whole tile before it when they fall in this head."""
    q_tiles = (cfg.S + BM - 1) // BM
    pick = {0, q_tiles // 2, q_tiles - 1}
    first_split = n_full - head_flat * q_tiles
    if 0 < first_split < q_tiles:
        pick |= {first_split - 1, first_split}
    return sorted(pick)


def _rows(cfg, tiles):
    return np.concatenate([np.arange(t * BM, min(cfg.S, (t + 1) * BM)) for t in tiles])


CASES = {  # config: kv heads sampled (one batch index, kv head index)
    "3": [(0, 0), (0, 39)],
    "4": [(0, 0), (0, 23)],
    "5a": [(0, 0), (1, 7)],
    "5b": [(0, 1), (1, 3)],
}


@pytest.mark.parametrize("name", list(CASES))
def test_config_full_workload(dev, name):
    cfg = CONFIGS[name]
    grp = cfg.H // cfg.Hkv
    q, k, v = make_inputs(cfg)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    res = sageattention.sageattn(qd, kd, vd, tensor_layout="HND", is_causal=cfg.causal, return_lse=cfg.return_lse)
    out, lse = (res if cfg.return_lse else (res, None))
    assert out.shape == q.shape and out.dtype == q.dtype
    n_full, chunks, _ = _capi.attn_plan(dev.index or 0, cfg.B, cfg.H, cfg.S, cfg.S, cfg.D, cfg.causal)
    skp = _capi.kv_pad(cfg.S)
    for b, hk in CASES[name]:
        heads = list(range(hk * grp, (hk + 1) * grp))
        hq = heads[0] if b == 0 else heads[-1]                  # one query head of the group
        # quantizers, bit-exact on the whole kv head and its query head at full length
        k1, v1 = k[b:b + 1, hk:hk + 1].contiguous(), v[b:b + 1, hk:hk + 1].contiguous()
        q1 = q[b:b + 1, hq:hq + 1].contiguous()
        kn, vn, qn = (t.float().numpy() for t in (k1, v1, q1))
        k8, ks, v8, vs = orc.quant_kv(kn, vn, seq_pad=skp)
        g_k8, g_ks, g_v8t, g_vs = run_quant_kv(k1.to(dev), v1.to(dev))
        assert np.array_equal(g_k8, k8) and np.array_equal(g_ks.view(np.uint32), ks.view(np.uint32))
        assert np.array_equal(g_vs.view(np.uint32), vs.view(np.uint32))
        assert np.array_equal(g_v8t, orc.v8_to_device_layout(v8))
        q8, qs = orc.quant_q(qn)
        g_q8, g_qs = run_quant_q(q1.to(dev))
        assert np.array_equal(g_q8, q8) and np.array_equal(g_qs.view(np.uint32), qs.view(np.uint32))
        # attention on sampled query tiles against the emulation at full key length
        head_flat = b * cfg.H + hq
        tiles = _tiles(cfg, n_full, head_flat)
        rows = _rows(cfg, tiles)
        split = kv_split(dev, cfg.B, cfg.H, cfg.S, cfg.S, cfg.D, cfg.causal, heads=[hq])
        if split is not None:
            split = (split[0], split[1][b:b + 1][:, :, rows])
        emu = orc.attention(np.ascontiguousarray(q8[:, :, rows]), np.ascontiguousarray(qs[:, :, rows]), k8, ks, v8,
                            vs, cfg.S, causal=cfg.causal, block_n=32, kv_split=split, q_rows=rows, seq_q=cfg.S,
                            also_unsplit=split is not None)
        emu, walk = emu if split is not None else (emu, None)
        got = out[b, hq][torch.from_numpy(rows).to(dev)].float().cpu().numpy()
        err = float(np.abs(got - emu[0, 0]).max())
        assert err <= MAX_ABS, (name, b, hq, err)
        if walk is not None and split[1].any():
            # rows of split tiles also against the reference's one walk over every key, with float64 attention
            # on the same rows for the outlier-scaled outputs of config 3
            sel = split[1][0, 0]
            ref = orc.sdpa_reference(qn[:, :, rows[sel]], kn, vn)[0, 0]
            gap = assert_near_walk(got[sel], walk[0, 0][sel], ref)
            print(f"config {name} b={b} head {hq}: {int(sel.sum())} split rows, max |out - walk| = {gap:.3g}",
                  flush=True)
        # cosine against float32 attention over the whole head
        cos = fp32_cos_head(qd[b, hq].float(), kd[b, hk].float(), vd[b, hk].float(), out[b, hq], cfg.causal)
        assert cos >= COS, (name, b, hq, cos)
        if lse is not None:
            qr = q1[0, 0, rows].double().numpy()
            kk = k1[0, 0].double().numpy()
            sc = qr @ kk.T * cfg.D ** -0.5
            if cfg.causal:
                sc = np.where(np.arange(cfg.S)[None, :] > rows[:, None], -np.inf, sc)
            mx = sc.max(-1)
            ref = mx + np.log(np.exp(sc - mx[:, None]).sum(-1))
            got_lse = lse[b, hq][torch.from_numpy(rows).to(dev)].double().cpu().numpy()
            assert np.all(np.abs(got_lse - ref) <= 2e-3 + 1e-4 * np.abs(ref)), (name, b, hq)
