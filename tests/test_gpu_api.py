"""The public API on the GPU, case for case after the reference's own tests (tests/test_attention.py,
tests/test_sageattention.py): kernel-forced shapes against float32 attention, sm_scale, SDPA routing, the
torch.library op under torch.compile, layouts / dtypes / causal, kernel-choice kwargs, return_lse and varlen.

Reference attention here is float32 torch matmul + softmax on the GPU, head by head, with GQA by repetition and a
bottom-right causal mask; transposed operands are made contiguous before every batched product."""
import math

import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

import cdna4_sage
import rdna4_sage
import sageattention

pytestmark = pytest.mark.gpu

COS = 0.998   # the reference's gate (tests/test_attention.py:54, tests/test_sageattention.py:14)


def ref_attention(q, k, v, layout="HND", causal=False, scale=None, heads=None):
    """float32 attention [B, H, Sq, D] (HND) computed per (batch, head); `heads` limits the query heads."""
    th = (lambda t: t) if layout == "HND" else (lambda t: t.transpose(1, 2))
    q, k, v = th(q), th(k), th(v)
    B, H, Sq, D = q.shape
    Skv, rep = k.shape[2], H // k.shape[1]
    scale = D ** -0.5 if scale is None else scale
    hs = range(H) if heads is None else heads
    out = torch.empty((B, len(hs), Sq, D), device=q.device, dtype=torch.float32)
    cols = torch.arange(Skv, device=q.device)
    for b in range(B):
        for n, h in enumerate(hs):
            kt = k[b, h // rep].float().t().contiguous()
            vf = v[b, h // rep].float().contiguous()
            for r0 in range(0, Sq, 4096):
                r1 = min(Sq, r0 + 4096)
                s = torch.matmul(q[b, h, r0:r1].float().contiguous(), kt) * scale
                if causal:
                    rows = torch.arange(r0, r1, device=q.device)[:, None] + (Skv - Sq)
                    s.masked_fill_(cols[None, :] > rows, float("-inf"))
                out[b, n, r0:r1] = torch.matmul(torch.softmax(s, dim=-1), vf)
    return out


def cos(a, b):
    return F.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0).item()


def rand(shape, dt, g, dev):
    return torch.randn(shape, generator=g).to(dt).to(dev)


# The reference's CASES (tests/test_attention.py:11-30): name, B, Sq, Skv, H, Hkv, D, layout, dtype[, causal]
REF_CASES = [
    ("SDXL self", 2, 4096, 4096, 10, 10, 64, "NHD", torch.float16),
    ("SD3.5 joint", 1, 4250, 4250, 24, 24, 64, "NHD", torch.float16),
    ("Flux joint", 1, 4352, 4352, 24, 24, 128, "HND", torch.bfloat16),
    ("Flux.2 joint", 1, 4608, 4608, 48, 48, 128, "HND", torch.bfloat16),
    ("Qwen-Image 1328", 1, 6889, 6889, 24, 24, 128, "HND", torch.bfloat16),
    ("Neta Lumina", 1, 4352, 4352, 24, 24, 96, "HND", torch.bfloat16),
    ("Lumina GQA 24/8", 1, 4096, 4096, 24, 8, 96, "HND", torch.bfloat16),
    ("Wan 1.3B 480p", 1, 32760, 32760, 12, 12, 128, "NHD", torch.float16),
    ("Wan cross 512", 1, 32760, 512, 12, 12, 128, "NHD", torch.float16),
    ("LTXV 2B", 1, 4992, 4992, 32, 32, 64, "NHD", torch.bfloat16),
    ("odd lengths", 3, 777, 1031, 6, 6, 128, "HND", torch.float16),
    ("AuraFlow joint d256", 1, 4360, 4360, 12, 12, 256, "HND", torch.float16),
    ("d256 odd lengths", 2, 777, 1031, 4, 4, 256, "NHD", torch.bfloat16),
    ("causal d128", 1, 4096, 4096, 24, 24, 128, "HND", torch.bfloat16, True),
    ("causal d64 odd", 2, 1000, 1000, 8, 8, 64, "NHD", torch.float16, True),
    ("causal d96 GQA 24/8", 1, 2048, 2048, 24, 8, 96, "HND", torch.bfloat16, True),
    ("causal d256", 1, 3000, 3000, 8, 8, 256, "NHD", torch.float16, True),
    ("causal d128 long", 1, 16384, 16384, 12, 12, 128, "HND", torch.bfloat16, True),
]


@pytest.mark.parametrize("case", REF_CASES, ids=[c[0] for c in REF_CASES])
def test_reference_cases(dev, case):
    name, B, Sq, Skv, H, Hkv, D, layout, dt, *c = case
    causal = bool(c and c[0])
    g = torch.Generator().manual_seed(0)
    shape = (lambda s, h: (B, h, s, D)) if layout == "HND" else (lambda s, h: (B, s, h, D))
    q, k, v = rand(shape(Sq, H), dt, g, dev), rand(shape(Skv, Hkv), dt, g, dev), rand(shape(Skv, Hkv), dt, g, dev)
    if D not in cdna4_sage.HEAD_DIMS:
        with pytest.raises(rdna4_sage.Unsupported):
            rdna4_sage.attention(q, k, v, tensor_layout=layout, is_causal=causal)
        return
    out = rdna4_sage.attention(q, k, v, tensor_layout=layout, is_causal=causal)   # kernel only, no routing
    assert out.dtype == dt and out.shape == q.shape
    heads = None if B * H * Sq * Skv <= 2**31 else [0, H - 1]                       # sample the largest cases
    ref = ref_attention(q, k, v, layout, causal, heads=heads)
    got = out if layout == "HND" else out.transpose(1, 2)
    if heads is not None:
        got = got[:, heads]
    assert cos(got, ref) > COS, (name, cos(got, ref))


def test_sm_scale_and_routing(dev):
    g = torch.Generator().manual_seed(1)
    q, k, v = (rand((1, 8, 2048, 128), torch.bfloat16, g, dev) for _ in range(3))
    ref = ref_attention(q, k, v, scale=0.05)
    assert cos(rdna4_sage.attention(q, k, v, "HND", sm_scale=0.05), ref) > COS
    # masked calls go to SDPA through the public drop-in (fp16 here: SDPA's masked bf16 path is avoided on this GPU)
    qh, kh, vh = (t.half() for t in (q, k, v))
    msk = torch.zeros(1, 1, 2048, 2048, device=dev, dtype=torch.float16)
    msk[..., :7] = float("-inf")
    torch.testing.assert_close(rdna4_sage.sageattn(qh, kh, vh, attn_mask=msk),
                               F.scaled_dot_product_attention(qh, kh, vh, attn_mask=msk))
    # causal with q_len < kv_len below MIN_WORK -> SDPA with a bottom-right mask
    qs = qh[:, :, :1500]
    keep = torch.ones(1500, 2048, dtype=torch.bool, device=dev).tril(2048 - 1500)
    torch.testing.assert_close(rdna4_sage.sageattn(qs, kh, vh, is_causal=True),
                               F.scaled_dot_product_attention(qs, kh, vh, attn_mask=keep))


def test_causal_q_shorter_than_kv_runs_the_kernel(dev):
    """Bottom-right causal with q_len < kv_len above MIN_WORK: the kernel (the reference sends it to SDPA with
    causal_lower_right), checked at the reference's gate against float32 attention with the same mask."""
    g = torch.Generator().manual_seed(4)
    q = rand((1, 24, 3000, 128), torch.bfloat16, g, dev)
    k, v = (rand((1, 24, 4096, 128), torch.bfloat16, g, dev) for _ in range(2))
    assert cdna4_sage._worth_it(q, k, "HND", True)
    out = sageattention.sageattn(q, k, v, is_causal=True)
    torch.testing.assert_close(out, cdna4_sage.attention(q, k, v, is_causal=True), rtol=0, atol=0)
    heads = [0, 13]
    assert cos(out[:, heads], ref_attention(q, k, v, causal=True, heads=heads)) > COS


def test_routed_call_uses_the_kernel(dev):
    """A call above MIN_WORK goes through the gfx950 kernel: bit-identical to the kernel-forced entry."""
    g = torch.Generator().manual_seed(2)
    q, k, v = (rand((1, 24, 4608, 128), torch.bfloat16, g, dev) for _ in range(3))
    assert cdna4_sage._worth_it(q, k, "HND")
    torch.testing.assert_close(sageattention.sageattn(q, k, v), cdna4_sage.attention(q, k, v), rtol=0, atol=0)
    small = q[:, :8, :1024, :64].contiguous()
    assert not cdna4_sage._worth_it(small, small, "HND")       # config 1 size stays on SDPA


def test_compile(dev):
    g = torch.Generator().manual_seed(3)
    q, k, v = (rand((1, 24, 4352, 128), torch.bfloat16, g, dev) for _ in range(3))
    f = torch.compile(lambda a, b, c: rdna4_sage.attention(a, b, c, "HND") * 2, fullgraph=True)
    torch.testing.assert_close(f(q, k, v), rdna4_sage.attention(q, k, v, "HND") * 2)
    f2 = torch.compile(lambda a, b, c: torch.ops.cdna4_sage.attention(a, b, c, "HND", 0.0, False), fullgraph=True)
    torch.testing.assert_close(f2(q, k, v), torch.ops.cdna4_sage.attention(q, k, v, "HND", 0.0, False))


@pytest.mark.parametrize("layout,dt,causal,D", [("HND", torch.bfloat16, False, 128), ("NHD", torch.float16, False, 64),
                                                ("HND", torch.float16, True, 128), ("NHD", torch.bfloat16, True, 96)])
def test_layouts_dtypes_causal(dev, layout, dt, causal, D):
    """tests/test_sageattention.py:38-46."""
    g = torch.Generator().manual_seed(4)
    shp = (1, 24, 4352, D) if layout == "HND" else (1, 4352, 24, D)
    q, k, v = (rand(shp, dt, g, dev) for _ in range(3))
    # keep any SDPA fallback off its unfused math path (bf16 batched products on transposed views)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        o = sageattention.sageattn(q, k, v, tensor_layout=layout, is_causal=causal)
    assert o.dtype == dt and o.shape == q.shape
    ref = ref_attention(q, k, v, layout, causal)
    assert cos(o if layout == "HND" else o.transpose(1, 2), ref) > COS


def test_variants_and_kwargs(dev):
    """tests/test_sageattention.py:49-59."""
    g = torch.Generator().manual_seed(5)
    q, k, v = (rand((2, 16, 4096, 128), torch.bfloat16, g, dev) for _ in range(3))
    r = ref_attention(q, k, v)
    for fn in (sageattention.sageattn_qk_int8_pv_fp16_triton, sageattention.sageattn_qk_int8_pv_fp16_cuda,
               sageattention.sageattn_qk_int8_pv_fp8_cuda, sageattention.sageattn_qk_int8_pv_fp8_cuda_sm90,
               sageattention.sageattn_qk_int8_pv_gfx12_native):
        assert cos(fn(q, k, v, tensor_layout="HND", smooth_k=True, pv_accum_dtype="fp32"), r) > COS, fn.__name__
    assert cos(sageattention.sageattn(q, k, v, is_causal=False, tensor_layout="HND", sm_scale=None, smooth_k=False), r) > COS
    assert cos(sageattention.sageattn(q, k, v, sm_scale=0.05), ref_attention(q, k, v, scale=0.05)) > COS


def test_return_lse(dev):
    """tests/test_sageattention.py:62-71: LSE [B, H, Sq] fp32 within atol 2e-3 / rtol 1e-4 of the float logits."""
    g = torch.Generator().manual_seed(6)
    q, k, v = (rand((1, 4, 2048, 64), torch.float16, g, dev) for _ in range(3))
    for causal in (False, True):
        o, lse = sageattention.sageattn(q, k, v, is_causal=causal, return_lse=True)
        sc = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * 64 ** -0.5
        if causal:
            sc.masked_fill_(torch.ones(2048, 2048, dtype=torch.bool, device=dev).triu(1), float("-inf"))
        assert lse.shape == (1, 4, 2048) and lse.dtype == torch.float32
        torch.testing.assert_close(lse, torch.logsumexp(sc, -1), atol=2e-3, rtol=1e-4)
        assert cos(o, ref_attention(q, k, v, causal=causal)) > COS


def test_varlen(dev):
    """tests/test_sageattention.py:74-84."""
    H, D, lens_q, lens_k = 8, 128, [3000, 1200, 2048], [3000, 512, 4096]
    cq = torch.tensor([0] + list(torch.tensor(lens_q).cumsum(0)), dtype=torch.int32, device=dev)
    ck = torch.tensor([0] + list(torch.tensor(lens_k).cumsum(0)), dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(7)
    q = rand((sum(lens_q), H, D), torch.bfloat16, g, dev)
    k, v = (rand((sum(lens_k), H, D), torch.bfloat16, g, dev) for _ in range(2))
    out = sageattention.sageattn_varlen(q, k, v, cq, ck, max(lens_q), max(lens_k))
    assert out.shape == q.shape
    for i in range(3):
        s = slice(int(cq[i]), int(cq[i + 1]))
        t = slice(int(ck[i]), int(ck[i + 1]))
        ref = ref_attention(q[None, s], k[None, t], v[None, t], "NHD")
        assert cos(out[s].transpose(0, 1)[None], ref) > COS, i


def _misaligned(t):
    """A contiguous copy of t whose base sits 4 elements (8 bytes) past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 8, device=t.device, dtype=t.dtype)
    u = buf[4:4 + t.numel()].view(t.shape)
    u.copy_(t)
    assert u.is_contiguous() and u.data_ptr() % 16 == 8
    return u


def test_misaligned_contiguous_inputs(dev):
    """Contiguous inputs on a base that is not 16-byte aligned (e.g. a view 4 elements into a buffer) are copied to
    an aligned tensor before the C call: the same bits as the aligned inputs, on the dense, LSE and varlen paths."""
    g = torch.Generator().manual_seed(11)
    q, k, v = (rand((1, 4, 1000, 128), torch.bfloat16, g, dev) for _ in range(3))
    want = cdna4_sage.attention(q, k, v, "HND", is_causal=True)
    got = cdna4_sage.attention(_misaligned(q), _misaligned(k), _misaligned(v), "HND", is_causal=True)
    assert torch.equal(got, want)
    assert torch.equal(cdna4_sage.lse(_misaligned(q), _misaligned(k), "HND", None, True),
                       cdna4_sage.lse(q, k, "HND", None, True))
    cu = torch.tensor([0, 700, 1000], dtype=torch.int32, device=dev)
    qp, kp, vp = (t[0].transpose(0, 1).contiguous() for t in (q, k, v))     # packed [tokens, heads, D]
    want = cdna4_sage.attention_varlen(qp, kp, vp, cu, cu, 700, 700)
    got = cdna4_sage.attention_varlen(_misaligned(qp), _misaligned(kp), _misaligned(vp), cu, cu, 700, 700)
    assert torch.equal(got, want)


def test_empty_inputs(dev):
    """An empty batch, no heads or no tokens: Unsupported from the kernel API (no C call); the routed API returns the
    empty output without calling torch SDPA, which raises for an empty batch on gfx950 and stops the process with
    SIGFPE for zero heads."""
    for shape_q, shape_kv in (((0, 4, 256, 128), (0, 4, 256, 128)), ((1, 0, 256, 128), (1, 0, 256, 128)),
                              ((1, 4, 0, 128), (1, 4, 256, 128)), ((1, 4, 256, 128), (1, 4, 0, 128))):
        q = torch.zeros(shape_q, device=dev, dtype=torch.bfloat16)
        k = torch.zeros(shape_kv, device=dev, dtype=torch.bfloat16)
        with pytest.raises(cdna4_sage.Unsupported):
            cdna4_sage.attention(q, k, k, "HND")
        if q.numel() == 0:
            out = sageattention.sageattn(q, k, k)
            assert out.shape == q.shape and out.dtype == q.dtype and out.device == q.device


def test_concurrent_streams_do_not_share_state(dev):
    """Entry points take their arguments by value: two streams running different problems at once give the same
    results as running them one after the other (the reference packs kernargs into one buffer per kernel)."""
    g = torch.Generator().manual_seed(8)
    a = [rand((1, 8, 2048, 128), torch.bfloat16, g, dev) for _ in range(3)]
    b = [rand((2, 4, 1500, 64), torch.float16, g, dev) for _ in range(3)]
    ra, rb = cdna4_sage.attention(*a), cdna4_sage.attention(*b)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(s1):
            oa = cdna4_sage.attention(*a)
        with torch.cuda.stream(s2):
            ob = cdna4_sage.attention(*b)
    torch.cuda.synchronize()
    torch.testing.assert_close(oa, ra, rtol=0, atol=0)
    torch.testing.assert_close(ob, rb, rtol=0, atol=0)
    assert math.isfinite(oa.float().abs().max().item())
