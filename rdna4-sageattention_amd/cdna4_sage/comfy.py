"""ComfyUI attention backend on the gfx950 kernels.

    import cdna4_sage.comfy
    cdna4_sage.comfy.register()   # ComfyUI's attention registry now lists "cdna4_sage"

A workflow picks a registered backend by name, per model (transformer_options["optimized_attention_override"]) or
as the preferred one (preferred_attention="cdna4_sage").  The reference registers the same function as "rdna4_sage"
(src/rdna4_sage/comfy.py:14-40); rdna4_sage.comfy.register() does that here.  Masked calls and calls with
low_precision_attention=False stay on ComfyUI's own PyTorch attention; the rest go through cdna4_sage.sageattn, whose
router sends small or unsupported shapes to SDPA.
"""
from comfy.ldm.modules.attention import attention_pytorch, register_attention_function, wrap_attn

from . import sageattn


@wrap_attn
def attention_cdna4_sage(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False, skip_output_reshape=False,
                         **kwargs):
    """ComfyUI's attention signature: q/k/v (B, L, heads * D), or (B, heads, L, D) with skip_reshape; the result is
    (B, L, heads * D), or (B, heads, L, D) with skip_output_reshape.  k / v may carry fewer heads (GQA)."""
    if mask is not None or kwargs.get("low_precision_attention", True) is False:
        return attention_pytorch(q, k, v, heads, mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                                 skip_output_reshape=skip_output_reshape, **kwargs)
    if skip_reshape:
        b, _, _, d = q.shape
        layout = "HND"
    else:
        b, _, width = q.shape
        d = width // heads
        # (B, L, H * D) -> (B, L, H, D) views; kv heads follow from k / v's own width
        q, k, v = q.unflatten(-1, (heads, d)), k.unflatten(-1, (-1, d)), v.unflatten(-1, (-1, d))
        layout = "NHD"
    out = sageattn(q, k, v, tensor_layout=layout, sm_scale=kwargs.get("scale"))
    if skip_output_reshape:
        return out if layout == "HND" else out.transpose(1, 2)
    return (out.transpose(1, 2) if layout == "HND" else out).reshape(b, -1, heads * d)


def register(name="cdna4_sage"):
    """Register the backend under `name` in ComfyUI's attention registry; returns the function."""
    register_attention_function(name, attention_cdna4_sage)
    return attention_cdna4_sage
