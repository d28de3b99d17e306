"""gfx950 LSE kernel (the row logsumexp `return_lse` returns) vs float64 on the CPU oracle and vs the reference's own
gate: atol 2e-3, rtol 1e-4 against fp32 torch (tests/test_sageattention.py:70 of the reference)."""
import os

import numpy as np
import pytest
import torch

import cdna4_sage
import sageattention
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

CASES = [  # B, H, Hkv, Sq, Skv, D, dtype, layout, causal
    (1, 2, 2, 300, 300, 128, torch.bfloat16, "HND", False),
    (2, 4, 2, 515, 515, 64, torch.float16, "NHD", False),
    (1, 4, 1, 257, 257, 64, torch.bfloat16, "HND", True),
    (1, 2, 2, 130, 777, 128, torch.float16, "HND", True),    # bottom-right causal with q_len < kv_len
    (3, 2, 2, 77, 1031, 128, torch.bfloat16, "NHD", False),
    (1, 3, 3, 1, 64, 128, torch.bfloat16, "HND", False),
    # short key ranges: the mask-free loop may run no tile at all
    (1, 2, 2, 96, 33, 128, torch.bfloat16, "HND", False),
    (1, 2, 2, 128, 128, 64, torch.float16, "NHD", True),
    (2, 2, 1, 70, 190, 128, torch.bfloat16, "HND", True),
    # 8 query heads per kv head (causal, batch 2) and multi-query
    (2, 16, 2, 600, 600, 128, torch.bfloat16, "HND", True),
    (1, 16, 1, 300, 900, 64, torch.float16, "NHD", False),
]


def _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, Sq, D, generator=g) * 1.5).to(dt)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
    if layout == "NHD":
        return q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    return q, k


def _hnd(t, layout):
    return (t if layout == "HND" else t.transpose(1, 2)).float().numpy()


@pytest.mark.parametrize("B,H,Hkv,Sq,Skv,D,dt,layout,causal", CASES)
def test_lse_vs_float64(dev, B, H, Hkv, Sq, Skv, D, dt, layout, causal):
    q, k = _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=Sq * 7 + Skv)
    got = cdna4_sage.lse(q.to(dev), k.to(dev), layout, None, causal).cpu().numpy()
    assert got.shape == (B, H, Sq) and got.dtype == np.float32
    ref = orc.lse_reference(_hnd(q, layout), _hnd(k, layout), causal=causal)
    # 16-bit products are exact in fp32; what remains is the fp32 accumulation order and exp2 / log2 (~1 ulp)
    assert np.abs(got - ref).max() <= 1e-4 + 1e-6 * np.abs(ref).max()


def test_lse_sm_scale_and_reference_gate(dev):
    """Config 5a shape on a sample (one kv group of 4 query heads, full sequence), explicit sm_scale, causal; checked
    at the reference's own tolerance against fp32 torch."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 4, 8192, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, 1, 8192, 128, generator=g).to(torch.bfloat16).to(dev)
    for causal in (False, True):
        got = cdna4_sage.lse(q, k, "HND", 0.07, causal)
        sc = torch.matmul(q.float(), k.float().repeat_interleave(4, 1).transpose(-1, -2).contiguous()) * 0.07
        if causal:
            sc.masked_fill_(torch.ones(8192, 8192, device=dev, dtype=torch.bool).triu(1), float("-inf"))
        torch.testing.assert_close(got, torch.logsumexp(sc, -1), atol=2e-3, rtol=1e-4)


def test_lse_unsupported_and_return_lse_uses_kernel(dev):
    q = torch.randn(1, 2, 100, 96, device=dev, dtype=torch.bfloat16)
    with pytest.raises(cdna4_sage.Unsupported):
        cdna4_sage.lse(q, q, "HND")
    q = torch.randn(1, 2, 300, 128, device=dev, dtype=torch.bfloat16)
    k = torch.randn(1, 2, 200, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(cdna4_sage.Unsupported):
        cdna4_sage.lse(q, k, "HND", None, True)                 # causal with q_len > kv_len: torch path instead
    v = torch.randn(1, 2, 2048, 128, device=dev, dtype=torch.bfloat16)
    q = torch.randn(1, 2, 2048, 128, device=dev, dtype=torch.bfloat16)
    k = torch.randn(1, 2, 2048, 128, device=dev, dtype=torch.bfloat16)
    _, lse = sageattention.sageattn(q, k, v, is_causal=True, return_lse=True)
    torch.testing.assert_close(lse, cdna4_sage.lse(q, k, "HND", None, True), atol=0, rtol=0)


def test_return_lse_side_stream_joins_the_callers_stream(dev):
    """sageattn(return_lse=True) computes the LSE on a side stream; work the caller queues on its own stream right
    after the call must see the finished LSE and output (the call joins the side stream before returning), also from a
    non-default caller stream, and the results equal the one-stream computation bit for bit."""
    g = torch.Generator().manual_seed(21)
    q = torch.randn(1, 8, 4096, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, 8, 4096, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(1, 8, 4096, 128, generator=g).to(torch.bfloat16).to(dev)
    ref_lse = cdna4_sage.lse(q, k, "HND", None, True)
    ref_out = sageattention.sageattn(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for _ in range(3):
            out, lse = sageattention.sageattn(q, k, v, is_causal=True, return_lse=True)
            lse_copy = lse * 1.0          # queued on the caller's stream right after the call
            out_copy = out.float() * 1.0
    s.synchronize()
    torch.testing.assert_close(lse_copy, ref_lse, atol=0, rtol=0)
    torch.testing.assert_close(out_copy, ref_out.float(), atol=0, rtol=0)


def test_return_lse_with_non_positive_sm_scale_uses_it_as_given(dev):
    """An explicit sm_scale <= 0 is taken as given by the reference's _lse (src/sageattention/core.py:31): the LSE
    kernel entry refuses it and the torch formula computes it, 0 giving log(kv_len)."""
    q, k = _inputs(1, 2, 2, 300, 1100, 128, torch.bfloat16, "HND", seed=9)
    qd, kd = q.to(dev), k.to(dev)
    with pytest.raises(cdna4_sage.Unsupported):
        cdna4_sage.lse(qd, kd, "HND", 0.0, False)
    for sm in (0.0, -0.05):
        _, lse = sageattention.sageattn(qd, kd, kd, tensor_layout="HND", sm_scale=sm, return_lse=True)
        s = torch.matmul(q.double(), k.double().transpose(-1, -2)) * sm
        torch.testing.assert_close(lse.cpu().double(), torch.logsumexp(s, -1), atol=2e-3, rtol=1e-4)
    _, lse0 = sageattention.sageattn(qd, kd, kd, tensor_layout="HND", sm_scale=0.0, return_lse=True)
    torch.testing.assert_close(lse0.cpu(), torch.full((1, 2, 300), float(np.log(1100.0))), atol=1e-4, rtol=0)


def _random_lse_cases(n=16, seed=4242):
    """Seeded random LSE shapes within the kernel's domain (D 64 or 128, causal only with q_len <= kv_len)."""
    rng = np.random.RandomState(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([64, 128]))
        Hkv = int(rng.randint(1, 4))
        H = Hkv * int(rng.choice([1, 2, 4]))
        B = int(rng.randint(1, 3))
        Skv = int(rng.choice([int(rng.randint(1, 130)), int(rng.randint(130, 1500))]))
        causal = bool(rng.rand() < 0.5)
        Sq = int(rng.randint(1, Skv + 1)) if causal else int(rng.randint(1, 700))
        dt = torch.bfloat16 if rng.rand() < 0.6 else torch.float16
        layout = "HND" if rng.rand() < 0.6 else "NHD"
        sm = None if rng.rand() < 0.7 else float(rng.uniform(0.03, 0.2))
        out.append((i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, sm))
    return out


RANDOM_LSE = _random_lse_cases(seed=4242 + int(os.environ.get("SAGE_SWEEP_SEED", "0")))


@pytest.mark.parametrize("case", RANDOM_LSE, ids=[
    f"{c[0]}-B{c[1]}H{c[2]}/{c[3]}-{c[4]}x{c[5]}-d{c[6]}-{c[8]}{'-causal' if c[9] else ''}{'-sm' if c[10] else ''}"
    for c in RANDOM_LSE])
def test_random_lse_vs_float64(dev, case):
    """Random shapes, GQA groups, layouts and scales against the float64 logsumexp, at the bound of the fixed cases."""
    i, B, H, Hkv, Sq, Skv, D, dt, layout, causal, sm = case
    q, k = _inputs(B, H, Hkv, Sq, Skv, D, dt, layout, seed=1000 + i)
    got = cdna4_sage.lse(q.to(dev), k.to(dev), layout, sm, causal).cpu().numpy()
    assert got.shape == (B, H, Sq) and np.isfinite(got).all()
    ref = orc.lse_reference(_hnd(q, layout), _hnd(k, layout), causal=causal, sm_scale=sm)
    assert np.abs(got - ref).max() <= 1e-4 + 1e-6 * np.abs(ref).max()


@pytest.mark.parametrize("causal", [False, True])
def test_lse_large_scales(dev, causal):
    """Inputs scaled by 100 (logits ~10^5): the running max moves rarely and by much; the float64 bound holds."""
    g = torch.Generator().manual_seed(77 + causal)
    q = (torch.randn(1, 2, 300, 128, generator=g) * 100).to(torch.bfloat16)
    k = (torch.randn(1, 2, 700, 128, generator=g) * 100).to(torch.bfloat16)
    got = cdna4_sage.lse(q.to(dev), k.to(dev), "HND", None, causal).cpu().numpy()
    ref = orc.lse_reference(_hnd(q, "HND"), _hnd(k, "HND"), causal=causal)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= 1e-4 + 1e-6 * np.abs(ref).max()
