"""The C ABI library without a GPU: it loads, exports every symbol include/sage_capi.h declares, describes itself
consistently with the committed manifest, and rejects invalid arguments with an error code and message before any
HIP call (so these checks run on a machine without a GPU)."""
import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

from cdna4_sage import _capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sage_capi.h"

pytestmark = pytest.mark.skipif(not _capi.LIB_PATH.exists(), reason="libsage_capi.so not built")

P = 0x10000  # a 16-byte-aligned fake device address; never dereferenced because validation fails first


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(sage_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = _capi.lib()
    names = declared_symbols()
    assert {"sage_quant_q", "sage_quant_kv", "sage_v_amax", "sage_attn_fwd", "sage_forward"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_capi.SIGNATURES), "ctypes signatures must cover exactly the header"


def test_abi_version_kv_pad_and_manifest():
    lib = _capi.lib()
    assert lib.sage_abi_version() == _capi.ABI_VERSION
    assert [_capi.kv_pad(s) for s in (1, 127, 128, 129, 4608, 67320)] == [128, 128, 128, 256, 4608, 67328]
    built = json.loads(lib.sage_manifest_json().decode())
    committed = json.loads((ROOT / "rdna4-sageattention_amd" / "cdna4_sage" / "manifest.json").read_text())
    assert {k: v for k, v in committed.items() if k not in ("library", "build_flags")} == built
    assert built["arch"] == "gfx950" and built["head_dims"] == [64, 96, 128, 256] and built["kv_block"] == 32


def _err():
    return _capi.lib().sage_last_error().decode()


def test_quant_q_validation():
    lib = _capi.lib()
    ok = (P, 128 * 64, 128, 64, 1, 2, 64, 128, 0, 1.0, P, P, None)   # noqa: F841 (shape of a valid call)
    assert lib.sage_quant_q(None, 0, 128, 0, 1, 1, 64, 128, 0, 1.0, P, P, None) == _capi.SAGE_ERR_INVALID
    assert "q is NULL" in _err()
    assert lib.sage_quant_q(P, 0, 128, 0, 1, 1, 64, 80, 0, 1.0, P, P, None) == _capi.SAGE_ERR_UNSUPPORTED
    assert "head_dim 80" in _err()
    assert [_capi.layout_dim(d) for d in (64, 96, 128, 256, 80, 0)] == [64, 128, 128, 256, 0, 0]
    assert lib.sage_quant_q(P + 2, 0, 128, 0, 1, 1, 64, 128, 0, 1.0, P, P, None) == _capi.SAGE_ERR_INVALID
    assert "aligned" in _err()
    assert lib.sage_quant_q(P, 0, 100, 0, 1, 1, 64, 128, 0, 1.0, P, P, None) == _capi.SAGE_ERR_INVALID
    assert "strides" in _err()
    assert lib.sage_quant_q(P, 0, 128, 0, 1, 1, 0, 128, 0, 1.0, P, P, None) == _capi.SAGE_ERR_INVALID
    assert lib.sage_quant_q(P, 0, 128, 0, 1, 1, 64, 128, 7, 1.0, P, P, None) == _capi.SAGE_ERR_UNSUPPORTED
    assert lib.sage_quant_q(P, 0, 128, 0, 1, 1, 64, 128, 0, 1.0, None, P, None) == _capi.SAGE_ERR_INVALID


def test_kv_and_attention_validation():
    lib = _capi.lib()
    assert lib.sage_v_amax(P, 0, 128, 0, 1, 1, 64, 128, 0, None, None) == _capi.SAGE_ERR_INVALID
    assert lib.sage_quant_kv(P, 0, 128, 0, P, 0, 128, 0, 1, 1, 64, 128, 0, P, P, P, P + 8, None) == _capi.SAGE_ERR_INVALID
    assert "16-byte" in _err()
    args = dict(q8=P, qs=P, k8=P, ks=P, v8t=P, vs=P, out=P, osb=0, oss=128, osh=128, B=1, H=4, Hkv=2, Sq=64, Skv=64,
                D=128, causal=0, out_dtype=0, lse=None, workspace=None, workspace_bytes=0, stream=None)

    def attn(**kw):
        a = dict(args, **kw)
        return lib.sage_attn_fwd(*a.values())

    assert attn(H=3) == _capi.SAGE_ERR_INVALID and "multiple" in _err()
    assert attn(causal=1, Sq=65) == _capi.SAGE_ERR_UNSUPPORTED and "q_len <= kv_len" in _err()
    assert attn(D=80) == _capi.SAGE_ERR_UNSUPPORTED
    assert attn(out_dtype=3) == _capi.SAGE_ERR_UNSUPPORTED
    assert attn(q8=None) == _capi.SAGE_ERR_INVALID
    assert attn(oss=100) == _capi.SAGE_ERR_INVALID
    assert attn(Sq=0) == _capi.SAGE_ERR_INVALID
    n_full, chunks, ws = ctypes.c_int(-1), ctypes.c_int(-1), ctypes.c_int64(-1)
    refs = (ctypes.byref(n_full), ctypes.byref(chunks), ctypes.byref(ws))
    assert lib.sage_attn_plan(1, 4, 64, 64, 80, 0, *refs) == _capi.SAGE_ERR_UNSUPPORTED and "head_dim 80" in _err()
    assert lib.sage_attn_plan(1, 4, 65, 64, 128, 1, *refs) == _capi.SAGE_ERR_UNSUPPORTED
    assert lib.sage_attn_plan(0, 4, 64, 64, 128, 0, *refs) == _capi.SAGE_ERR_INVALID
    assert (n_full.value, chunks.value, ws.value) == (-1, -1, -1)       # outputs untouched on error
    wsb = ctypes.c_int64(-1)
    assert lib.sage_forward_workspace(1, 4, 3, 64, 64, 128, 0, ctypes.byref(wsb)) == _capi.SAGE_ERR_INVALID
    assert lib.sage_forward_workspace(1, 4, 2, 64, 64, 128, 0, None) == _capi.SAGE_ERR_INVALID


def test_forward_validates_before_launching_and_python_raises():
    lib = _capi.lib()
    rc = lib.sage_forward(P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 128, 1, 4, 2, 80, 64, 128, 0, 1, 1.0,
                          P, P, P, P, P, P, None, 0, None)
    assert rc == _capi.SAGE_ERR_UNSUPPORTED and "causal" in _err()
    with pytest.raises(_capi.SageError, match="head_dim 80"):
        _capi.call("sage_quant_q", P, 0, 128, 0, 1, 1, 64, 80, 0, 1.0, P, P, None)


@pytest.mark.parametrize("qs_mul", [0.0, -1.0, float("nan"), float("inf")])
def test_qs_mul_must_be_positive_and_finite(qs_mul):
    # the attention takes its row maxima on the raw integer scores, which needs positive row scales
    lib = _capi.lib()
    assert lib.sage_quant_q(P, 0, 128, 0, 1, 1, 64, 128, 0, qs_mul, P, P, None) == _capi.SAGE_ERR_INVALID
    assert "qs_mul" in _err()
    rc = lib.sage_forward(P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 128, 1, 4, 2, 64, 64, 128, 0, 0, qs_mul,
                          P, P, P, P, P, P, None, 0, None)
    assert rc == _capi.SAGE_ERR_INVALID and "qs_mul" in _err()
    rc = lib.sage_forward_noalloc(P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 128, 1, 4, 2, 64, 64, 128, 0, 0,
                                  qs_mul, None)
    assert rc == _capi.SAGE_ERR_INVALID and "qs_mul" in _err()


@pytest.mark.parametrize("bad, what", [("k", "k is not 16-byte aligned"), ("kss", "strides"), ("q", "q is NULL")])
def test_forward_without_workspace_checks_q_k_v_first(bad, what):
    # without a workspace sage_forward's first launch takes the V maxima; a bad q or k must be rejected before it
    # (here, with no GPU, a launch would fail with a HIP error instead of the argument error)
    lib = _capi.lib()
    a = dict(q=P, qsb=0, qss=128, qsh=0, k=P, ksb=0, kss=128, ksh=0, v=P, vsb=0, vss=128, vsh=0)
    a.update({"k": P + 8} if bad == "k" else {"kss": 100} if bad == "kss" else {"q": None})
    rc = lib.sage_forward(*a.values(), P, 0, 128, 128, 1, 4, 2, 64, 64, 128, 0, 0, 1.0, P, P, P, P, P, P, None, 0, None)
    assert rc == _capi.SAGE_ERR_INVALID, _err()
    assert what in _err()


@pytest.mark.parametrize("bad, what", [("out", "pointer argument is NULL"), ("out_align", "16-byte aligned"),
                                       ("oss", "out strides"), ("q8", "pointer argument is NULL"),
                                       ("v8t", "16-byte aligned"), ("skv", "too long")])
@pytest.mark.parametrize("with_ws", [False, True])
def test_forward_checks_the_attention_arguments_before_launching(bad, what, with_ws):
    # the output, the intermediates and the attention's size limits are checked before the quantizers launch (with no
    # GPU here, a launch would fail with a HIP error instead of the argument error)
    lib = _capi.lib()
    skv = 2**24 if bad == "skv" else 64  # 128 channels x 2^24 keys: past the 2^31-byte V8T head the kernels index
    inputs = (P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 0)
    out = None if bad == "out" else P + 8 if bad == "out_align" else P
    osb, oss, osh = 0, (100 if bad == "oss" else 128), 128
    inter = [P] * 6
    if bad == "q8":
        inter[0] = None
    if bad == "v8t":
        inter[4] = P + 4
    ws, ws_bytes = (P, 1 << 40) if with_ws else (None, 0)
    rc = lib.sage_forward(*inputs, out, osb, oss, osh, 1, 4, 2, 64, skv, 128, 0, 0, 1.0, *inter, ws, ws_bytes, None)
    assert rc == _capi.SAGE_ERR_INVALID, _err()
    assert what in _err(), _err()


def test_varlen_layout_bounds():
    """Padded key rows: sum of the sequences' lengths rounded up to 128 is at most total + 127 * batch; query tiles:
    sum of ceil(len / 128) is at most (total + 127 * batch) / 128.  Tables are 256-byte aligned regions."""
    lib = _capi.lib()
    rows, ws = ctypes.c_int(-1), ctypes.c_int64(-1)
    assert lib.sage_varlen_layout(3, 4, 2, 300, 500, ctypes.byref(rows), ctypes.byref(ws)) == _capi.SAGE_OK
    assert rows.value == (500 + 127 * 3) // 128 * 128 == 768
    # header, kp, order, tpre, ktab: one 256-byte region each; tiles: 4 heads x 5 query tiles x 16 bytes -> 512
    assert ws.value == 5 * 256 + 512
    assert _capi.varlen_layout(3, 4, 2, 300, 500) == (768, 1792)
    rng = np.random.default_rng(0)
    for _ in range(200):
        batch = int(rng.integers(1, 40))
        lk = rng.integers(0, 3000, batch)
        lq = rng.integers(0, 3000, batch)
        tk, tq = int(lk.sum()) + 1, int(lq.sum()) + 1
        r, _ = _capi.varlen_layout(batch, 8, 2, tq, tk)
        assert r % 128 == 0 and int(((lk + 127) // 128 * 128).sum()) <= r
        tiles = int(((lq + 127) // 128).sum())
        assert tiles <= (tq + 127 * batch) // 128
    assert lib.sage_varlen_layout(0, 4, 2, 300, 500, None, None) == _capi.SAGE_ERR_INVALID
    assert lib.sage_varlen_layout(2, 4, 3, 300, 500, None, None) == _capi.SAGE_ERR_INVALID and "multiple" in _err()
    assert lib.sage_varlen_layout(2, 4, 2, 300, 0, None, None) == _capi.SAGE_ERR_INVALID
    assert lib.sage_varlen_layout(1, 4, 2, 300, 2**24, None, None) == _capi.SAGE_ERR_INVALID and "too large" in _err()


def test_varlen_validates_before_launching():
    lib = _capi.lib()
    _, ws_bytes = _capi.varlen_layout(2, 4, 2, 256, 256)
    args = dict(q=P, qss=512, qsh=128, k=P, kss=256, ksh=128, v=P, vss=256, vsh=128, out=P, oss=512, osh=128,
                cu_q=P, cu_k=P, batch=2, H=4, Hkv=2, total_q=256, total_k=256, D=128, dtype=0, causal=1, qs_mul=1.0,
                q8=P, qs=P, k8=P, ks=P, v8t=P, vs=P, ws=P, ws_bytes=ws_bytes, stream=None)

    def call(**kw):
        a = dict(args, **kw)
        return lib.sage_forward_varlen(*a.values())

    assert call(D=80) == _capi.SAGE_ERR_UNSUPPORTED and "head_dim 80" in _err()
    assert call(dtype=2) == _capi.SAGE_ERR_UNSUPPORTED
    assert call(Hkv=3) == _capi.SAGE_ERR_INVALID
    assert call(q=P + 8) == _capi.SAGE_ERR_INVALID and "16-byte" in _err()
    assert call(kss=100) == _capi.SAGE_ERR_INVALID and "multiples of 8" in _err()
    assert call(cu_k=None) == _capi.SAGE_ERR_INVALID and "cu_seqlens" in _err()
    assert call(v8t=None) == _capi.SAGE_ERR_INVALID
    assert call(ws_bytes=ws_bytes - 1) == _capi.SAGE_ERR_INVALID and "workspace" in _err()
    assert call(ws=P + 16) == _capi.SAGE_ERR_INVALID and "256-byte" in _err()
    assert call(qs_mul=float("nan")) == _capi.SAGE_ERR_INVALID and "qs_mul" in _err()
    assert call(total_q=0) == _capi.SAGE_ERR_INVALID


def test_masked_forward_validates_before_launching():
    """sage_forward_masked / sage_mask_workspace reject bad shapes, strides and pointers with a code and a message
    before the first HIP call (on this GPU-less machine any later step would fail with a HIP error instead)."""
    lib = _capi.lib()
    args = dict(q=P, qsb=0, qss=128, qsh=0, k=P, ksb=0, kss=128, ksh=0, v=P, vsb=0, vss=128, vsh=0, out=P, osb=0,
                oss=128, osh=128, B=1, H=4, Hkv=2, Sq=80, Skv=200, D=128, dtype=0, causal=0, qs_mul=1.0,
                mask=P, mask_dtype=_capi.DTYPE_BOOL, msb=0, msh=0, msq=200, q8=P, qs=P, k8=P, ks=P, v8t=P, vs=P, ws=P,
                ws_bytes=1 << 30, stream=None)

    def call(**kw):
        a = dict(args, **kw)
        return lib.sage_forward_masked(*a.values())

    assert call(D=80) == _capi.SAGE_ERR_UNSUPPORTED and "head_dim 80" in _err()
    assert call(causal=1, Sq=300) == _capi.SAGE_ERR_UNSUPPORTED and "causal" in _err()
    assert call(Hkv=3) == _capi.SAGE_ERR_INVALID and "multiple" in _err()
    assert call(msq=-1) == _capi.SAGE_ERR_INVALID and "mask strides" in _err()
    assert call(dtype=5) == _capi.SAGE_ERR_UNSUPPORTED
    assert call(mask=None) == _capi.SAGE_ERR_INVALID and "mask is NULL" in _err()
    assert call(out=P + 8) == _capi.SAGE_ERR_INVALID and "out" in _err()
    assert call(oss=100) == _capi.SAGE_ERR_INVALID and "multiples of 8" in _err()
    assert call(ws=None) == _capi.SAGE_ERR_INVALID and "workspace" in _err()
    assert call(ws=P + 16) == _capi.SAGE_ERR_INVALID and "256-byte" in _err()
    assert call(qs_mul=-0.5) == _capi.SAGE_ERR_INVALID and "qs_mul" in _err()
    assert call(Sq=1 << 20, Skv=1 << 30) == _capi.SAGE_ERR_INVALID and "too large" in _err()
    assert call(mask_dtype=7) == _capi.SAGE_ERR_UNSUPPORTED and "mask dtype" in _err()
    assert call(mask_dtype=_capi.DTYPE_F16) == _capi.SAGE_ERR_UNSUPPORTED and "inputs' dtype" in _err()
    # the bias values of an additive mask make its per-(batch, head) tables 16x larger than a bool mask's
    assert call(mask_dtype=_capi.DTYPE_BF16, Sq=1 << 18, Skv=1 << 17) == _capi.SAGE_ERR_INVALID and "too large" in _err()
    ws = ctypes.c_int64(-1)
    B = _capi.DTYPE_BOOL
    assert lib.sage_mask_workspace(1, 4, 2, 80, 200, 96, 1, B, 0, 0, -5, ctypes.byref(ws)) == _capi.SAGE_ERR_INVALID
    assert lib.sage_mask_workspace(1, 4, 2, 80, 200, 80, 0, B, 0, 0, 0, ctypes.byref(ws)) == _capi.SAGE_ERR_UNSUPPORTED
    assert lib.sage_mask_workspace(1, 4, 2, 80, 200, 128, 0, B, 0, 0, 0, None) == _capi.SAGE_ERR_INVALID
    assert ws.value == -1


def test_forward_noalloc_rejects_before_touching_the_gpu():
    """sage_forward_noalloc validates shapes like sage_forward and refuses a shape whose intermediates and workspace
    exceed its static scratch array (causal shapes plan without querying the device, so this runs without a GPU)."""
    lib = _capi.lib()
    args = (P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 0, P, 0, 128, 128)
    rc = lib.sage_forward_noalloc(*args, 1, 4, 2, 80, 64, 128, 0, 1, 1.0, None)
    assert rc == _capi.SAGE_ERR_UNSUPPORTED and "causal" in _err()
    rc = lib.sage_forward_noalloc(*args, 1, 4, 2, 64, 64, 80, 0, 0, 1.0, None)
    assert rc == _capi.SAGE_ERR_UNSUPPORTED and "head_dim 80" in _err()
    rc = lib.sage_forward_noalloc(*args, 1, 40, 40, 32760, 32760, 128, 0, 1, 1.0, None)
    assert rc == _capi.SAGE_ERR_INVALID and "scratch" in _err() and str(128 << 20) in _err()
    # the array's own size: 128 MiB, the value the header states
    assert "(128ll << 20)" in HEADER.read_text()


def test_bench_intermediates_have_the_abi_layout_sizes():
    """bench.py hands its own Q8 / QS / K8 / KS / V8T / VS to sage_forward and sage_attn_fwd, which cannot check
    buffer sizes: every configuration's buffers must have the sizes of include/sage_capi.h's layouts (int8 / E4M3
    rows of 128 channels for head dim 96, keys padded to 128).  Head-dim-sized buffers for the d96 configuration were
    written past their end on the GPU."""
    import bench
    from cdna4_sage.configs import CONFIGS

    for name, cfg in CONFIGS.items():
        B, H, Hkv, S, D = cfg.B, cfg.H, cfg.Hkv, cfg.S, cfg.D
        dl = 128 if D == 96 else D
        skp = (S + 127) // 128 * 128
        want = [B * H * S * dl, 4 * B * H * S, B * Hkv * skp * dl, 4 * B * Hkv * skp // 32, B * Hkv * dl * skp,
                4 * B * Hkv * dl]
        got = [t.numel() * t.element_size() for t in bench.intermediates(cfg, "meta")]
        assert got == want, (name, got, want)
