"""ComfyUI backend (cdna4_sage.comfy, rdna4_sage.comfy; reference: src/rdna4_sage/comfy.py:14-40) against a stand-in
of ComfyUI's attention registry.  On the CPU every call routes to SDPA, which checks the reshapes and the fallback
rules; the kernel path is covered by tests/test_gpu_comfy.py."""
import importlib

import pytest
import torch
import torch.nn.functional as F

import comfy_stub


@pytest.fixture(scope="module")
def comfy():
    comfy_stub.install()
    import cdna4_sage.comfy
    import rdna4_sage.comfy
    importlib.reload(cdna4_sage.comfy)
    importlib.reload(rdna4_sage.comfy)
    return cdna4_sage.comfy, rdna4_sage.comfy


def _ref(q, k, v, scale=None):   # (B, H, L, D) float32 reference
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=k.shape[1] != q.shape[1],
                                          scale=scale)


def test_register_names(comfy):
    c, r = comfy
    assert c.register() is c.attention_cdna4_sage and comfy_stub.REGISTRY["cdna4_sage"] is c.attention_cdna4_sage
    assert r.register() is c.attention_cdna4_sage and "rdna4_sage" in comfy_stub.REGISTRY
    c.register("custom")
    assert "custom" in comfy_stub.REGISTRY


@pytest.mark.parametrize("hkv", [4, 2])
def test_reshape_contract(comfy, hkv):
    c, _ = comfy
    g = torch.Generator().manual_seed(0)
    B, H, L, D = 2, 4, 50, 64
    q = torch.randn(B, H, L, D, generator=g)
    k = torch.randn(B, hkv, 70, D, generator=g)
    v = torch.randn(B, hkv, 70, D, generator=g)
    ref = _ref(q, k, v)
    flat = lambda t: t.transpose(1, 2).reshape(B, t.shape[2], -1)   # noqa: E731  (B, L, heads * D)
    out = c.attention_cdna4_sage(flat(q), flat(k), flat(v), H)
    assert out.shape == (B, L, H * D)
    torch.testing.assert_close(out, flat(ref), atol=1e-5, rtol=1e-5)
    out = c.attention_cdna4_sage(q, k, v, H, skip_reshape=True)
    torch.testing.assert_close(out, flat(ref), atol=1e-5, rtol=1e-5)
    out = c.attention_cdna4_sage(q, k, v, H, skip_reshape=True, skip_output_reshape=True)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    out = c.attention_cdna4_sage(flat(q), flat(k), flat(v), H, skip_output_reshape=True)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    out = c.attention_cdna4_sage(q, k, v, H, skip_reshape=True, skip_output_reshape=True, scale=0.05)
    torch.testing.assert_close(out, _ref(q, k, v, 0.05), atol=1e-5, rtol=1e-5)


def test_mask_and_low_precision_opt_out_use_comfy_attention(comfy):
    c, _ = comfy
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 40, 64, generator=g) for _ in range(3))
    mask = torch.zeros(40, 40)
    mask[:, :3] = float("-inf")
    comfy_stub.CALLS.clear()
    out = c.attention_cdna4_sage(q, k, v, 2, mask=mask, skip_reshape=True, skip_output_reshape=True)
    torch.testing.assert_close(out, F.scaled_dot_product_attention(q, k, v, attn_mask=mask))
    c.attention_cdna4_sage(q, k, v, 2, skip_reshape=True, low_precision_attention=False)
    assert comfy_stub.CALLS == ["pytorch", "pytorch"]
    c.attention_cdna4_sage(q, k, v, 2, skip_reshape=True)
    assert comfy_stub.CALLS == ["pytorch", "pytorch"]          # the sageattn route
