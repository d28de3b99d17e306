"""A stand-in for the three names ComfyUI's attention registry exposes (comfy.ldm.modules.attention), installed into
sys.modules so that cdna4_sage.comfy imports without ComfyUI.  attention_pytorch follows ComfyUI's reshape contract:
(B, L, heads * D) in and out, (B, heads, L, D) with skip_reshape / skip_output_reshape."""
import sys
import types

import torch
import torch.nn.functional as F

REGISTRY = {}
CALLS = []


def attention_pytorch(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False, skip_output_reshape=False,
                      **kwargs):
    CALLS.append("pytorch")
    if skip_reshape:
        b, _, _, d = q.shape
    else:
        b, _, width = q.shape
        d = width // heads
        q, k, v = (t.view(b, -1, t.shape[-1] // d, d).transpose(1, 2) for t in (q, k, v))
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=k.shape[1] != q.shape[1],
                                         scale=kwargs.get("scale"))
    return out if skip_output_reshape else out.transpose(1, 2).reshape(b, -1, heads * d)


def register_attention_function(name, fn):
    REGISTRY[name] = fn


def wrap_attn(fn):
    return fn


def install():
    mod = types.ModuleType("comfy.ldm.modules.attention")
    mod.attention_pytorch = attention_pytorch
    mod.register_attention_function = register_attention_function
    mod.wrap_attn = wrap_attn
    for name in ("comfy", "comfy.ldm", "comfy.ldm.modules"):
        sys.modules.setdefault(name, types.ModuleType(name))
    sys.modules["comfy.ldm.modules.attention"] = mod
    return mod
