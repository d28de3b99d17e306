"""ComfyUI backend on the gfx950 kernels: the registered function gives exactly what sageattn gives for the same
call, in ComfyUI's (B, L, heads * D) contract and with skip_reshape / skip_output_reshape."""
import importlib

import pytest
import torch

import cdna4_sage
import comfy_stub

pytestmark = pytest.mark.gpu


def test_comfy_backend_runs_the_kernel(dev):
    comfy_stub.install()
    import cdna4_sage.comfy
    importlib.reload(cdna4_sage.comfy)
    fn = cdna4_sage.comfy.register()
    g = torch.Generator().manual_seed(0)
    B, H, L, D = 1, 24, 4608, 128
    q, k, v = (torch.randn(B, L, H * D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    assert cdna4_sage._worth_it(q.view(B, L, H, D), k.view(B, L, H, D), "NHD")
    comfy_stub.CALLS.clear()
    out = fn(q, k, v, H)
    direct = cdna4_sage.sageattn(q.view(B, L, H, D), k.view(B, L, H, D), v.view(B, L, H, D), tensor_layout="NHD")
    assert torch.equal(out, direct.reshape(B, L, H * D)) and not comfy_stub.CALLS
    hnd = [t.view(B, L, H, D).transpose(1, 2) for t in (q, k, v)]
    out2 = fn(*hnd, H, skip_reshape=True, skip_output_reshape=True)
    torch.testing.assert_close(out2, cdna4_sage.sageattn(*hnd, tensor_layout="HND"), rtol=0, atol=0)
    ref = torch.nn.functional.scaled_dot_product_attention(*(t[:, :2].float() for t in hnd))
    cos = torch.nn.functional.cosine_similarity(out2[:, :2].float().flatten(), ref.flatten(), dim=0).item()
    assert cos >= 0.998
