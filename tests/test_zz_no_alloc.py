"""sage_forward_noalloc (intermediates and workspace in the library's static device array) against sage_forward with
caller-owned buffers: the same kernels on the same plan, so the outputs must be equal bit for bit.  Two calls in a
row on one GPU, the second with a smaller problem, so the second runs on what the first left in the array."""
import ctypes

import numpy as np
import pytest
import torch

from cdna4_sage import _capi

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: _capi.DTYPE_BF16, torch.float16: _capi.DTYPE_F16}


def _inputs(B, H, Hkv, S, D, dt, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, S, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, S, D, generator=g).to(dt)
    return q, k, v


def _hnd(t):
    return t.stride(0), t.stride(2), t.stride(1)


def _forward(q, k, v, causal, noalloc):
    dev = q.device
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(B, S, H, D, dtype=q.dtype, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    head = (q.data_ptr(), *_hnd(q), k.data_ptr(), *_hnd(k), v.data_ptr(), *_hnd(v), out.data_ptr(),
            out.stride(0), out.stride(1), out.stride(2), B, H, Hkv, S, S, D, DT[q.dtype], int(causal), 1.0)
    if noalloc:
        _capi.call("sage_forward_noalloc", *head, st)
    else:
        dl, skp = _capi.layout_dim(D), _capi.kv_pad(S)
        bufs = [torch.empty(B, H, S, dl, dtype=torch.int8, device=dev), torch.empty(B, H, S, device=dev),
                torch.empty(B, Hkv, skp, dl, dtype=torch.int8, device=dev), torch.empty(B, Hkv, skp // 32, device=dev),
                torch.empty(B, Hkv, dl, skp, dtype=torch.uint8, device=dev), torch.empty(B, Hkv, dl, device=dev)]
        ws_bytes = _capi.forward_workspace(dev.index or 0, B, H, Hkv, S, S, D, bool(causal))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _capi.call("sage_forward", *head, *(b.data_ptr() for b in bufs), ws.data_ptr(), ws_bytes, st)
    torch.cuda.synchronize(dev)
    return out


def test_noalloc_matches_sage_forward_on_consecutive_calls(dev):
    cases = [  # B, H, Hkv, S, D, dtype, causal: the second is smaller than the first
        (1, 8, 4, 2000, 128, torch.bfloat16, False),
        (1, 4, 2, 333, 64, torch.float16, True),
        (2, 6, 6, 1100, 256, torch.bfloat16, False),
    ]
    for i, (B, H, Hkv, S, D, dt, causal) in enumerate(cases):
        q, k, v = (t.to(dev) for t in _inputs(B, H, Hkv, S, D, dt, seed=100 + i))
        ref = _forward(q, k, v, causal, noalloc=False)
        got = _forward(q, k, v, causal, noalloc=True)
        assert torch.equal(got, ref), (i, float((got.float() - ref.float()).abs().max()))
        assert bool(torch.isfinite(got).all())


def test_noalloc_rejects_a_shape_beyond_its_array(dev):
    q = torch.empty(1, 40, 32760, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_capi.SageError, match="scratch"):
        _capi.call("sage_forward_noalloc", q.data_ptr(), *_hnd(q), q.data_ptr(), *_hnd(q), q.data_ptr(), *_hnd(q),
                   q.data_ptr(), 0, 128, 128, 1, 40, 40, 32760, 32760, 128, 0, 0, 1.0,
                   torch.cuda.current_stream(dev).cuda_stream)


def _noalloc_call(q, k, v, out):
    """sage_forward_noalloc on torch's current stream, no synchronisation (so that it can be captured)."""
    B, H, S, D = q.shape
    _capi.call("sage_forward_noalloc", q.data_ptr(), *_hnd(q), k.data_ptr(), *_hnd(k), v.data_ptr(), *_hnd(v),
               out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), B, H, k.shape[1], S, S, D, DT[q.dtype], 0,
               1.0, torch.cuda.current_stream(q.device).cuda_stream)


def test_noalloc_replays_under_graph_capture(dev):
    """After one eager call on the GPU (which looks up the array's address), a captured sage_forward_noalloc replays
    bit-equal to sage_forward, also when an eager call with another, smaller problem ran on the same array between
    the replays (the replay recomputes every intermediate)."""
    B, H, Hkv, S, D = 1, 8, 4, 1500, 128
    q, k, v = (t.to(dev) for t in _inputs(B, H, Hkv, S, D, torch.bfloat16, seed=41))
    ref = _forward(q, k, v, False, noalloc=False)
    out = torch.empty(B, S, H, D, dtype=q.dtype, device=dev)
    _noalloc_call(q, k, v, out)                                     # eager, before the capture
    torch.cuda.synchronize(dev)
    assert torch.equal(out, ref)
    q2, k2, v2 = (t.to(dev) for t in _inputs(1, 4, 2, 700, 64, torch.float16, seed=42))
    ref2 = _forward(q2, k2, v2, False, noalloc=False)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _noalloc_call(q, k, v, out)
    for i in range(3):
        out.fill_(3.0)
        got2 = _forward(q2, k2, v2, False, noalloc=True)            # another problem on the same array, eager
        assert torch.equal(got2, ref2), i
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, ref), i
