"""Bit-exact parity of the gfx950 quantizers with the CPU oracle (int8 Q/K, E4M3 V and every scale)."""
import numpy as np
import pytest
import torch

from gpu_util import DT as DT_CODE
from gpu_util import bits, hnd_np, run_quant_kv, run_quant_q, unpad
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

Q_CASES = [  # B, H, S, D, dtype, layout
    (1, 2, 100, 128, torch.bfloat16, "HND"),
    (2, 3, 777, 64, torch.float16, "NHD"),
    (1, 4, 1, 128, torch.bfloat16, "HND"),
    (1, 2, 4099, 64, torch.bfloat16, "NHD"),
    (2, 5, 130, 128, torch.float16, "HND"),
    (1, 24, 4608, 128, torch.bfloat16, "HND"),   # config 2 (Flux) at full size
    (1, 3, 333, 96, torch.bfloat16, "NHD"),      # no rotation, stored as 128 channels
    (2, 2, 129, 256, torch.float16, "HND"),      # two 128-channel Hadamard blocks
]


def _randn(shape, dtype, seed, layout="HND", scale=1.0):
    g = torch.Generator().manual_seed(seed)
    B, H, S, D = shape
    t = torch.randn(B, H, S, D, generator=g) * scale
    t = t.to(dtype)
    return t if layout == "HND" else t.transpose(1, 2).contiguous()


@pytest.mark.parametrize("B,H,S,D,dt,layout", Q_CASES)
def test_quant_q_bitexact(dev, B, H, S, D, dt, layout):
    q = _randn((B, H, S, D), dt, 11 + S, layout)
    q8, qs = run_quant_q(q.to(dev), layout)
    q8 = unpad(q8, D)
    e8, es = orc.quant_q(hnd_np(q, layout))
    assert np.array_equal(q8, e8), f"Q8 mismatch at {np.argwhere(q8 != e8)[:5]}"
    assert np.array_equal(bits(qs), bits(es))


def test_quant_q_sm_scale_fold(dev):
    q = _randn((1, 2, 300, 128), torch.bfloat16, 5)
    f = orc.qs_fold_factor(0.05, 128)
    _, qs = run_quant_q(q.to(dev), "HND", float(f))
    _, es = orc.quant_q(hnd_np(q), sm_scale=0.05)
    assert np.array_equal(bits(qs), bits(es))


KV_CASES = [  # B, Hkv, S, D, dtype, layout
    (1, 2, 100, 128, torch.bfloat16, "HND"),
    (2, 3, 777, 64, torch.float16, "NHD"),
    (1, 1, 1, 128, torch.bfloat16, "HND"),
    (1, 2, 1031, 64, torch.bfloat16, "HND"),
    (2, 2, 257, 128, torch.float16, "NHD"),
    (1, 24, 4608, 128, torch.bfloat16, "HND"),   # config 2 (Flux) at full size
    (2, 2, 300, 96, torch.float16, "HND"),
    (1, 3, 777, 256, torch.bfloat16, "NHD"),
]


@pytest.mark.parametrize("B,H,S,D,dt,layout", KV_CASES)
def test_quant_kv_bitexact(dev, B, H, S, D, dt, layout):
    k = _randn((B, H, S, D), dt, 21 + S, layout)
    v = _randn((B, H, S, D), dt, 31 + S, layout, scale=2.0)
    k8, ks, v8t, vs = run_quant_kv(k.to(dev), v.to(dev), layout)
    k8, v8t, vs = unpad(k8, D), unpad(v8t, D, axis=2), unpad(vs, D)
    skp = k8.shape[2]
    e8, eks, ev8, evs = orc.quant_kv(hnd_np(k, layout), hnd_np(v, layout), seq_pad=skp)
    assert np.array_equal(bits(vs), bits(evs)), "VS mismatch"
    assert np.array_equal(k8, e8), f"K8 mismatch at {np.argwhere(k8 != e8)[:5]}"
    assert np.array_equal(bits(ks), bits(eks)), "KS mismatch"
    ev8t = orc.v8_to_device_layout(ev8)
    assert np.array_equal(v8t, ev8t), f"V8T mismatch at {np.argwhere(v8t != ev8t)[:5]}"


def test_quant_edge_values(dev):
    """Zero rows, a zero V channel, outlier channels, wide exponent spread and fp16 subnormals."""
    for dt in (torch.bfloat16, torch.float16):
        g = torch.Generator().manual_seed(3)
        S, D = 200, 128
        k = torch.randn(1, 2, S, D, generator=g)
        v = torch.randn(1, 2, S, D, generator=g)
        k[:, :, 5] = 0.0                       # a zero row (scale clamps at 1e-12)
        k[:, :, 7, 3] = 300.0                  # one outlier
        k[:, 1, 40:72] = 0.0                   # a whole zero K block
        v[:, :, :, 9] = 0.0                    # a zero V channel
        v[:, 0, :, 17] *= 1000.0 if dt == torch.bfloat16 else 100.0
        k[:, :, 100] *= 1e-3
        if dt == torch.float16:
            k[:, :, 120] = torch.randn(1, 2, D, generator=g) * 2.0**-20   # fp16 subnormals
            v[:, :, 121] = torch.randn(1, 2, D, generator=g) * 2.0**-20
        else:
            k[:, :, 120] *= 2.0**-60
            v[:, :, 121] *= 2.0**-60
        k, v = k.to(dt), v.to(dt)
        q8, qs = run_quant_q(k.to(dev))
        e8, es = orc.quant_q(hnd_np(k))
        assert np.array_equal(q8, e8) and np.array_equal(bits(qs), bits(es)), dt
        k8, ks, v8t, vs = run_quant_kv(k.to(dev), v.to(dev))
        ek8, eks, ev8, evs = orc.quant_kv(hnd_np(k), hnd_np(v), seq_pad=k8.shape[2])
        assert np.array_equal(k8, ek8) and np.array_equal(bits(ks), bits(eks)), dt
        assert np.array_equal(bits(vs), bits(evs)), dt
        assert np.array_equal(v8t, orc.v8_to_device_layout(ev8)), dt


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_quant_v_e4m3_rounding_points(dev, dt):
    """V values on every E4M3 code, every midpoint between neighbours (ties to even), one input ulp either side of
    each midpoint, and the subnormal range, both signs.  Channels 0-63 have amax 448 (scale exactly 1, so the
    conversion sees these values as they are); channels 64-127 are scaled by 0.37, so it sees arbitrary float32
    neighbours of them.  The kernel's E4M3 bytes must equal the oracle's round-to-nearest-even."""
    codes = orc.e4m3_to_f32(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (codes[:-1] + codes[1:]) / 2
    cand = np.concatenate([codes, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9),
                           np.arange(1, 64) * 2.0 ** -12, [2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -11]])
    col = torch.from_numpy(cand).float().to(dt)
    col = torch.unique(torch.cat([col, -col]))
    S = col.numel() + 1
    v = torch.empty(1, 1, S, 128, dtype=torch.float32)
    v[0, 0, 0] = 448.0
    v[0, 0, 1:] = col.float()[:, None]
    v[..., 64:] *= 0.37
    v = v.to(dt)
    k = _randn((1, 1, S, 128), dt, 77)
    k8, ks, v8t, vs = run_quant_kv(k.to(dev), v.to(dev))
    _, _, ev8, evs = orc.quant_kv(hnd_np(k), hnd_np(v), seq_pad=k8.shape[2])
    assert np.array_equal(bits(vs), bits(evs))
    ev8t = orc.v8_to_device_layout(ev8)
    bad = np.argwhere(v8t != ev8t)
    assert bad.size == 0, f"{len(bad)} E4M3 mismatches, first at {bad[:5]}"


FWD_CASES = [  # B, H, Hkv, S, D, dtype
    (1, 2, 2, 1000, 128, torch.bfloat16),
    (2, 4, 2, 515, 64, torch.float16),
    (1, 3, 1, 77, 128, torch.bfloat16),
    (1, 24, 24, 4608, 128, torch.bfloat16),   # config 2 (Flux): 9 chunks of V maxima
    (1, 4, 2, 600, 96, torch.bfloat16),
    (1, 2, 2, 1100, 256, torch.float16),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,dt", FWD_CASES)
@pytest.mark.parametrize("with_workspace", [True, False])
def test_forward_intermediates_bitexact(dev, B, H, Hkv, S, D, dt, with_workspace):
    """sage_forward's own intermediates: with a workspace the quantizers run fused (Q + per-chunk V maxima in one
    launch, K / V reducing the maxima in the next), without one as four launches; both must equal the oracle."""
    from cdna4_sage import _capi
    q = _randn((B, H, S, D), dt, 3 + S).to(dev)
    k = _randn((B, Hkv, S, D), dt, 4 + S).to(dev)
    v = _randn((B, Hkv, S, D), dt, 5 + S, scale=3.0).to(dev)
    skp = _capi.kv_pad(S)
    dl = _capi.layout_dim(D)
    q8 = torch.full((B, H, S, dl), 5, dtype=torch.int8, device=dev)      # stale values must be overwritten
    qs = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    k8 = torch.full((B, Hkv, skp, dl), 5, dtype=torch.int8, device=dev)
    ks = torch.empty(B, Hkv, skp // 32, dtype=torch.float32, device=dev)
    v8t = torch.full((B, Hkv, dl, skp), 5, dtype=torch.uint8, device=dev)
    vs = torch.full((B, Hkv, dl), 7.0, dtype=torch.float32, device=dev)
    out = torch.empty(B, S, H, D, dtype=dt, device=dev)
    wsb = _capi.forward_workspace(dev.index or 0, B, H, Hkv, S, S, D, False) if with_workspace else 0
    ws = torch.full((max(wsb, 1),), 0xFF, dtype=torch.uint8, device=dev)
    hnd = lambda t: (t.stride(0), t.stride(2), t.stride(1))  # noqa: E731
    _capi.call("sage_forward", q.data_ptr(), *hnd(q), k.data_ptr(), *hnd(k), v.data_ptr(), *hnd(v), out.data_ptr(),
               out.stride(0), out.stride(1), out.stride(2), B, H, Hkv, S, S, D, DT_CODE[dt], 0, 1.0, q8.data_ptr(),
               qs.data_ptr(), k8.data_ptr(), ks.data_ptr(), v8t.data_ptr(), vs.data_ptr(),
               ws.data_ptr() if with_workspace else None, wsb, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    eq8, eqs = orc.quant_q(hnd_np(q.cpu()))
    ek8, eks, ev8, evs = orc.quant_kv(hnd_np(k.cpu()), hnd_np(v.cpu()), seq_pad=skp)
    assert np.array_equal(unpad(q8.cpu().numpy(), D), eq8) and np.array_equal(bits(qs.cpu().numpy()), bits(eqs))
    assert np.array_equal(bits(unpad(vs.cpu().numpy(), D)), bits(evs)), "VS mismatch"
    assert np.array_equal(unpad(k8.cpu().numpy(), D), ek8) and np.array_equal(bits(ks.cpu().numpy()), bits(eks))
    assert np.array_equal(unpad(v8t.cpu().numpy(), D, axis=2), orc.v8_to_device_layout(ev8)), "V8T mismatch"
    assert torch.isfinite(out.float()).all()
