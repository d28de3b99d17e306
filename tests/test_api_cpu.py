"""Host-side behaviour that needs no GPU: API surface, SDPA routing, the torch.library op's fake implementation,
the return_lse path and varlen, checked against the reference's documented semantics
(src/sageattention/core.py, src/rdna4_sage/__init__.py, tests/test_sageattention.py)."""
import inspect
import os
import subprocess
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cdna4_sage
import rdna4_sage
import sageattention
from oracle import sage_oracle as orc

VARIANTS = ["sageattn_qk_int8_pv_fp16_triton", "sageattn_qk_int8_pv_fp16_cuda", "sageattn_qk_int8_pv_fp8_cuda",
            "sageattn_qk_int8_pv_fp8_cuda_sm90", "sageattn_qk_int8_pv_gfx12_native"]


def _rand(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def test_api_surface():
    for n in ["sageattn", "sageattn_varlen"] + VARIANTS:
        assert callable(getattr(sageattention, n)), n
    # ComfyUI decides mask support from the signature: SageAttention 2.2's sageattn has no attn_mask parameter
    assert "attn_mask" not in inspect.signature(sageattention.sageattn).parameters
    params = {n: list(inspect.signature(getattr(sageattention, n)).parameters) for n in VARIANTS}
    assert params["sageattn_qk_int8_pv_fp16_triton"][:5] == ["q", "k", "v", "tensor_layout", "quantization_backend"]
    assert "attn_mask" in params["sageattn_qk_int8_pv_fp16_triton"]
    assert "qk_quant_gran" in params["sageattn_qk_int8_pv_fp8_cuda"] and "pv_accum_dtype" in params["sageattn_qk_int8_pv_fp8_cuda"]
    assert "value_dtype" in params["sageattn_qk_int8_pv_gfx12_native"]
    vp = inspect.signature(sageattention.sageattn_varlen).parameters
    assert list(vp)[:7] == ["q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k"]
    for mod in (cdna4_sage, rdna4_sage):
        for n in ["sageattn", "attention", "is_available", "Unsupported", "ARCHS", "HEAD_DIMS"]:
            assert hasattr(mod, n), (mod, n)
    assert cdna4_sage.ARCHS == ("gfx950",) and cdna4_sage.HEAD_DIMS == (64, 96, 128, 256)
    assert hasattr(torch.ops.cdna4_sage, "attention") and hasattr(torch.ops.rdna4_sage, "attention")


@pytest.mark.parametrize("layout", ["HND", "NHD"])
@pytest.mark.parametrize("causal", [False, True])
def test_cpu_tensors_route_to_sdpa(layout, causal):
    q, k, v = (_rand((1, 4, 300, 64), s, torch.bfloat16) for s in (1, 2, 3))
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    th = (lambda t: t) if layout == "HND" else (lambda t: t.transpose(1, 2))
    out = sageattention.sageattn(q, k, v, tensor_layout=layout, is_causal=causal)
    ref = th(F.scaled_dot_product_attention(th(q), th(k), th(v), is_causal=causal))
    assert out.shape == q.shape and out.dtype == q.dtype
    torch.testing.assert_close(out, ref, rtol=0, atol=0)


def test_kernel_forced_api_raises_unsupported_on_cpu():
    q = _rand((1, 2, 64, 64), 4, torch.bfloat16)
    with pytest.raises(cdna4_sage.Unsupported):
        cdna4_sage.attention(q, q, q, "HND")
    with pytest.raises(rdna4_sage.Unsupported):
        rdna4_sage.attention(q, q, q, "HND")
    with pytest.raises(cdna4_sage.Unsupported, match="layout"):
        cdna4_sage.check_supported(q, q, q, "BHSD")
    with pytest.raises(NotImplementedError):
        cdna4_sage.sageattn(q, q, q, return_lse=True)


def test_causal_q_len_ne_kv_len_is_bottom_right():
    q = _rand((1, 2, 30, 64), 5)
    k, v = _rand((1, 2, 50, 64), 6), _rand((1, 2, 50, 64), 7)
    keep = torch.ones(30, 50, dtype=torch.bool).tril(50 - 30)
    torch.testing.assert_close(sageattention.sageattn(q, k, v, is_causal=True),
                               F.scaled_dot_product_attention(q, k, v, attn_mask=keep))


def test_mask_and_gqa_go_to_sdpa():
    q = _rand((1, 8, 40, 64), 8)
    k, v = _rand((1, 2, 40, 64), 9), _rand((1, 2, 40, 64), 10)
    m = torch.zeros(1, 1, 40, 40)
    m[..., :5] = float("-inf")
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), attn_mask=m)
    torch.testing.assert_close(sageattention.sageattn(q, k, v, attn_mask=m), ref)
    torch.testing.assert_close(sageattention.sageattn(q, k, v),
                               F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1)))


def test_worth_it_thresholds_and_env_names():
    q = torch.empty(1, 24, 4608, 128, device="meta")
    assert cdna4_sage._worth_it(q, q, "HND")
    small = torch.empty(1, 8, 1024, 64, device="meta")                # config 1: 8.4 M < 64 Mi -> SDPA
    assert not cdna4_sage._worth_it(small, small, "HND")
    short = torch.empty(1, 64, 2048, 64, device="meta")
    kshort = torch.empty(1, 64, 512, 64, device="meta")              # kv shorter than MIN_KV -> SDPA
    assert not cdna4_sage._worth_it(short, kshort, "HND")
    code = "import sys; sys.path.insert(0, sys.argv[1]); import cdna4_sage as c; print(c.MIN_WORK, c.MIN_KV)"
    pkg = os.path.join(os.path.dirname(__file__), "..", "rdna4-sageattention_amd")
    for env, want in [({"RDNA4_SAGE_MIN_WORK": "5", "RDNA4_SAGE_MIN_KV": "7"}, "5 7"),
                      ({"CDNA4_SAGE_MIN_WORK": "9", "RDNA4_SAGE_MIN_WORK": "5"}, "9 1024")]:
        e = {k: v for k, v in os.environ.items() if "SAGE_MIN" not in k}
        e.update(env)
        out = subprocess.run([sys.executable, "-c", code, pkg], env=e, capture_output=True, text=True, check=True)
        assert out.stdout.strip() == want


def test_fake_impl_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 24, 100, 128, dtype=torch.bfloat16)
        kv = torch.empty(2, 8, 300, 128, dtype=torch.bfloat16)
        assert torch.ops.cdna4_sage.attention(q, kv, kv, "HND", 0.0, False).shape == (2, 100, 24, 128)
        qn = torch.empty(2, 100, 24, 64, dtype=torch.float16)
        kvn = torch.empty(2, 300, 8, 64, dtype=torch.float16)
        o = torch.ops.rdna4_sage.attention(qn, kvn, kvn, "NHD", 0.0, False)
        assert o.shape == (2, 100, 24, 64) and o.dtype == torch.float16
        # the Python entry points route fake tensors through the registered ops (their eager shortcut is for plain
        # tensors only), so tracers see the fake implementation
        assert not cdna4_sage._plain_eager(q, kv, kv)
        assert cdna4_sage.attention(q, kv, kv, "HND").shape == (2, 24, 100, 128)
        assert rdna4_sage.attention(qn, kvn, kvn, "NHD").shape == (2, 100, 24, 64)
    assert cdna4_sage._plain_eager(torch.empty(1), torch.empty(1))


@pytest.mark.parametrize("layout", ["HND", "NHD"])
@pytest.mark.parametrize("causal", [False, True])
def test_return_lse_matches_float64(layout, causal):
    """LSE semantics of src/sageattention/core.py:23-44 (unquantized fp32, bottom-right causal, GQA) against a
    float64 logsumexp; the reference's gate is atol 2e-3, rtol 1e-4 (tests/test_sageattention.py:70)."""
    q = _rand((1, 4, 70, 64), 11, torch.float16)
    k, v = _rand((1, 2, 90, 64), 12, torch.float16), _rand((1, 2, 90, 64), 13, torch.float16)
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    if causal:                                  # causal q_len != kv_len is bottom-right aligned
        pass
    out, lse = sageattention.sageattn(q, k, v, tensor_layout=layout, is_causal=causal, return_lse=True)
    th = (lambda t: t) if layout == "HND" else (lambda t: t.transpose(1, 2))
    ref = orc.lse_reference(th(q).float().numpy(), th(k).float().numpy(), causal=causal)
    assert lse.shape == (1, 4, 70) and lse.dtype == torch.float32
    np.testing.assert_allclose(lse.numpy(), ref, atol=2e-3, rtol=1e-4)
    assert out.shape == q.shape


def test_invalid_layout_in_lse_raises_value_error():
    q = _rand((1, 2, 8, 64), 14)
    with pytest.raises(ValueError):
        sageattention.core._lse(q, q, "BSHD", False, None)


def test_variants_accept_and_ignore_kernel_kwargs():
    q, k, v = (_rand((1, 2, 64, 64), s) for s in (15, 16, 17))
    ref = sageattention.sageattn(q, k, v)
    for n in VARIANTS:
        out = getattr(sageattention, n)(q, k, v, tensor_layout="HND", smooth_k=True, pv_accum_dtype="fp32")
        torch.testing.assert_close(out, ref, rtol=0, atol=0)
    o, lse = sageattention.sageattn_qk_int8_pv_fp8_cuda(q, k, v, return_lse=True)
    assert lse.shape == (1, 2, 64)


def test_varlen_matches_per_sequence_attention():
    H, D = 4, 64
    lq, lk = [30, 0, 45, 12], [30, 20, 70, 5]
    cq = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32)
    ck = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32)
    q = _rand((sum(lq), H, D), 18)
    k, v = _rand((sum(lk), H, D), 19), _rand((sum(lk), H, D), 20)
    for causal in (False, True):
        out = sageattention.sageattn_varlen(q, k, v, cq, ck, max(lq), max(lk), is_causal=causal)
        assert out.shape == q.shape
        for i in range(len(lq)):
            s, t = slice(int(cq[i]), int(cq[i + 1])), slice(int(ck[i]), int(ck[i + 1]))
            if lq[i] == 0:
                continue
            qq, kk, vv = (x.transpose(0, 1)[None] for x in (q[s], k[t], v[t]))
            if causal:
                keep = torch.ones(lq[i], lk[i], dtype=torch.bool).tril(lk[i] - lq[i])
                ref = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=keep)
            else:
                ref = F.scaled_dot_product_attention(qq, kk, vv)
            torch.testing.assert_close(out[s], ref[0].transpose(0, 1))


def test_mask_view_strides_and_rejections():
    """The mask as the kernel reads it: broadcast axes at stride 0, the key axis contiguous (materialised alone when
    it is not), element strides of (batch, head, row), the dtype code (bool, or an additive mask of q's dtype);
    masks of another dtype and non-broadcastable masks are rejected."""
    from cdna4_sage import _capi
    from cdna4_sage._attention import Unsupported, mask_view
    q = torch.zeros(2, 4, 6, 64, dtype=torch.bfloat16)   # HND: B=2, H=4, Sq=6
    k = torch.zeros(2, 2, 10, 64, dtype=torch.bfloat16)  # Skv=10
    pad = torch.ones(2, 1, 1, 10, dtype=torch.bool)
    m, code, st = mask_view(pad, q, k, "HND")
    assert m.shape == (2, 4, 6, 10) and st == (10, 0, 0) and m.data_ptr() == pad.data_ptr()
    assert code == _capi.DTYPE_BOOL
    m, code, st = mask_view(torch.ones(6, 10, dtype=torch.bool), q, k, "HND")
    assert st == (0, 0, 10)
    m, code, st = mask_view(torch.ones(10, dtype=torch.bool), q.transpose(1, 2), k.transpose(1, 2), "NHD")
    assert st == (0, 0, 0)
    full = torch.rand(2, 4, 10, 6) > 0.5
    m, code, st = mask_view(full.transpose(2, 3), q, k, "HND")       # key axis not contiguous: materialised
    assert m.stride(3) == 1 and torch.equal(m, full.transpose(2, 3)) and st == (240, 60, 10)
    col = torch.rand(2, 1, 6, 1) > 0.5                           # broadcast over keys: only the key axis is filled in
    m, code, st = mask_view(col, q, k, "HND")
    assert m.stride(3) == 1 and st == (60, 0, 10) and torch.equal(m, col.expand(2, 4, 6, 10))
    bias = torch.randn(1, 4, 6, 10).to(torch.bfloat16)           # additive mask of q's dtype
    m, code, st = mask_view(bias, q, k, "HND")
    assert code == _capi.DTYPE_BF16 and st == (0, 60, 10) and m.dtype == torch.bfloat16
    m, code, st = mask_view(torch.zeros(6, 10, dtype=torch.float16), q.half(), k.half(), "HND")
    assert code == _capi.DTYPE_F16
    for bad in (torch.zeros(6, 10), torch.zeros(6, 10, dtype=torch.float16), torch.ones(3, 1, 6, 10, dtype=torch.bool),
                torch.ones(1, 1, 1, 1, 10, dtype=torch.bool)):
        with pytest.raises(Unsupported):
            mask_view(bad, q, k, "HND")


def test_bool_mask_routing_without_kernel_uses_sdpa():
    """On a machine without a gfx950 GPU a boolean mask still takes the SDPA path (check_supported fails first), with
    the causal mask ANDed in bottom-right aligned."""
    import cdna4_sage
    q, k, v = (torch.randn(1, 2, 8, 64) for _ in range(3))
    mask = torch.rand(1, 1, 8, 8) > 0.3
    mask[..., 0] = True
    out = cdna4_sage.sageattn(q, k, v, attn_mask=mask)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    assert torch.allclose(out, ref, atol=1e-6)


@pytest.mark.parametrize("B,H,Hkv,Sq,Skv,D", [(1, 24, 24, 4608, 4608, 128), (2, 32, 8, 8192, 8192, 64),
                                             (3, 2, 2, 77, 1031, 96), (1, 3, 1, 1, 1, 256)])
def test_single_block_layouts(monkeypatch, B, H, Hkv, Sq, Skv, D):
    """The dense and varlen paths carve Q8, QS, K8, KS, V8T, VS and the workspace out of one allocation: every piece
    starts on a 256-byte boundary, none overlaps the next, and each is as large as the library's layout needs
    (the workspace sizes come from the library's plan queries, which need a GPU; stand-ins here)."""
    from cdna4_sage import _attention, _capi

    monkeypatch.setattr(_capi, "forward_workspace", lambda *a: 12345)
    monkeypatch.setattr(_capi, "varlen_layout", lambda batch, H_, Hkv_, TQ, TK: ((TK // 128 + batch) * 128, 777))
    _attention._forward_layout.cache_clear()
    _attention._varlen_layout.cache_clear()
    skp, dl = _capi.kv_pad(Skv), _capi.layout_dim(D)
    offs, total, ws, skp_, dl_ = _attention._forward_layout(0, B, H, Hkv, Sq, Skv, D, False)
    assert (skp_, dl_, ws) == (skp, dl, 12345)
    need = [B * H * Sq * dl, B * H * Sq * 4, B * Hkv * skp * dl, B * Hkv * skp // 32 * 4, B * Hkv * dl * skp,
            B * Hkv * dl * 4, 12345]
    ends = [o + n for o, n in zip(offs, need)]
    assert all(o % 256 == 0 for o in offs)
    assert all(e <= o for e, o in zip(ends, offs[1:])) and ends[-1] <= total
    TQ, TK = B * Sq, B * Skv
    voffs, vtotal, vws = _attention._varlen_layout(B, H, Hkv, TQ, TK, D)
    tkp = (TK // 128 + B) * 128
    vneed = [H * TQ * dl, H * TQ * 4, Hkv * tkp * dl, Hkv * tkp // 32 * 4, Hkv * dl * tkp, B * Hkv * dl * 4, 777]
    vends = [o + n for o, n in zip(voffs, vneed)]
    assert vws == 777 and all(o % 256 == 0 for o in voffs)
    assert all(e <= o for e, o in zip(vends, voffs[1:])) and vends[-1] <= vtotal
    _attention._forward_layout.cache_clear()
    _attention._varlen_layout.cache_clear()


def test_autograd_inputs_reach_the_registered_op(monkeypatch):
    """With inputs that require grad, the Python entry points go through the registered op (not the eager shortcut),
    whose output autograd tracks; backward then raises for the missing derivative, as for the reference's op."""
    from cdna4_sage import ops

    q = torch.randn(1, 2, 16, 64, dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(1, 2, 16, 64, dtype=torch.bfloat16)
    assert not cdna4_sage._plain_eager(q, k, k)
    with torch.no_grad():
        assert cdna4_sage._plain_eager(q, k, k)
    calls = []
    monkeypatch.setattr(ops, "_impl", lambda q_, k_, v_, layout, sm, causal: calls.append(1) or
                        torch.zeros(q_.shape[0], q_.shape[2], q_.shape[1], q_.shape[3], dtype=q_.dtype))
    monkeypatch.setattr(cdna4_sage, "_attention_impl", lambda *a, **kw: pytest.fail("eager shortcut taken"))
    out = cdna4_sage.attention(q, k, k, "HND")
    assert calls and out.requires_grad
    with pytest.raises(RuntimeError):
        out.float().sum().backward()


def test_lse_with_non_positive_sm_scale_uses_it_as_given():
    """The reference's _lse multiplies by an explicit sm_scale as given (src/sageattention/core.py:31), 0 and negative
    values included; the LSE kernel entry leaves such scales to the torch formula."""
    q = _rand((1, 2, 20, 64), 31)
    k = _rand((1, 2, 40, 64), 32)
    for sm in (0.0, -0.1):
        lse = sageattention.core._lse(q, k, "HND", False, sm)
        s = torch.matmul(q.double(), k.double().transpose(-1, -2)) * sm
        torch.testing.assert_close(lse.double(), torch.logsumexp(s, -1), atol=2e-3, rtol=1e-4)


def test_qs_fold_factor_maps_non_positive_scales_to_the_default():
    """The attention's scale fold (the dense, masked and packed varlen passes all use it): None, the default 1/sqrt(D),
    0, negative values and NaN fold nothing, as the reference's op maps sm_scale <= 0 to None
    (src/rdna4_sage/ops.py:10); any other positive scale folds sm_scale * sqrt(D), as the oracle does."""
    from cdna4_sage._attention import qs_fold_factor
    for sm in (None, 128 ** -0.5, 0.0, -0.25, float("nan")):
        assert qs_fold_factor(sm, 128) == 1.0
        assert orc.qs_fold_factor(sm, 128) is None
    for sm, d in ((0.05, 128), (0.3, 64), (1.0, 96)):
        assert qs_fold_factor(sm, d) == pytest.approx(sm * d ** 0.5, rel=1e-12)
        assert np.float32(qs_fold_factor(sm, d)) == orc.qs_fold_factor(sm, d)


def test_bsh_strides_and_the_copy_rule():
    """(batch, seq, head) element strides handed to the quantizers (reference: src/rdna4_sage/_attention.py:59-67):
    views whose strides are multiples of 8 elements and whose base is 16-byte aligned pass through uncopied, in
    both layouts; anything else is made contiguous first."""
    from cdna4_sage._attention import _bsh
    x = torch.zeros(2, 3, 40, 64, dtype=torch.bfloat16)                  # HND [B, H, S, D]
    t, st = _bsh(x, "HND")
    assert t.data_ptr() == x.data_ptr() and st == (3 * 40 * 64, 64, 40 * 64)
    t, st = _bsh(x, "NHD")                                                # read as [B, S, H, D]
    assert t.data_ptr() == x.data_ptr() and st == (3 * 40 * 64, 40 * 64, 64)
    y = x.transpose(1, 2)                                                 # NHD view of the HND tensor
    t, st = _bsh(y, "NHD")
    assert t.data_ptr() == x.data_ptr() and st == (3 * 40 * 64, 64, 40 * 64)
    z = torch.zeros(2, 3, 40, 72, dtype=torch.bfloat16)[..., :64]        # row stride 72: a multiple of 8, kept
    t, st = _bsh(z, "HND")
    assert t.data_ptr() == z.data_ptr() and st == (3 * 40 * 72, 72, 40 * 72)
    w = torch.zeros(2, 3, 40, 68, dtype=torch.bfloat16)[..., :64]        # row stride 68: copied
    t, st = _bsh(w, "HND")
    assert t.is_contiguous() and st == (3 * 40 * 64, 64, 40 * 64)
    u = torch.zeros(2 * 3 * 40 * 64 + 8, dtype=torch.bfloat16)[4:4 + 2 * 3 * 40 * 64].view(2, 3, 40, 64)
    assert u.data_ptr() % 16 == 8
    t, st = _bsh(u, "HND")                                                # 8-byte aligned base: copied
    assert t.data_ptr() != u.data_ptr() and t.data_ptr() % 16 == 0 and st == (3 * 40 * 64, 64, 40 * 64)
    v = x[..., ::2]                                                       # channel stride 2: copied
    t, st = _bsh(v, "HND")
    assert t.is_contiguous() and st == (3 * 40 * 32, 32, 40 * 32)


def test_return_lse_with_empty_inputs():
    """No query rows (empty batch, no heads, no tokens): the output and the logsumexp come back empty, with
    [batch, heads, q_len] for the latter."""
    for shape in ((0, 2, 16, 64), (1, 0, 16, 64), (1, 2, 0, 64)):
        q = torch.zeros(shape)
        k = torch.zeros(shape[:2] + (16, 64))
        out, lse = sageattention.sageattn(q, k, k, return_lse=True)
        assert out.shape == q.shape and lse.shape == shape[:3] and lse.dtype == torch.float32
