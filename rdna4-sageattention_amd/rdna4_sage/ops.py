"""torch.ops.rdna4_sage.attention: the reference's op name (src/rdna4_sage/ops.py:7-17), same schema and fake impl,
served by the gfx950 kernels of cdna4_sage."""
import torch

from cdna4_sage import ops as _ops


@torch.library.custom_op("rdna4_sage::attention", mutates_args=())
def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: str, sm_scale: float, is_causal: bool) -> torch.Tensor:
    """Output [batch, q_len, heads, head_dim], contiguous, whatever the input layout; a non-positive sm_scale stands
    for the default 1 / sqrt(head_dim)."""
    return _ops._impl(q, k, v, layout, sm_scale, is_causal)


attention.register_fake(_ops._fake)
