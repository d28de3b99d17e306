"""torch.library registration: torch.ops.cdna4_sage.attention (and attention_masked), traceable by torch.compile.

Same schema as the reference's rdna4_sage::attention (src/rdna4_sage/ops.py:7-17); the rdna4_sage package of this
repo registers that name too, for callers that use it directly.
"""
import torch

from . import _attention


def _impl(q, k, v, layout, sm_scale, is_causal):
    return _attention.attention(q, k, v, layout, sm_scale if sm_scale > 0 else None, is_causal)


def _fake(q, k, v, layout, sm_scale, is_causal):
    B = q.shape[0]
    H, Sq = (q.shape[1], q.shape[2]) if layout == "HND" else (q.shape[2], q.shape[1])
    return q.new_empty((B, Sq, H, q.shape[3]))


@torch.library.custom_op("cdna4_sage::attention", mutates_args=())
def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: str, sm_scale: float, is_causal: bool) -> torch.Tensor:
    """Output [batch, q_len, heads, head_dim], contiguous, whatever the input layout; a non-positive sm_scale stands
    for the default 1 / sqrt(head_dim)."""
    return _impl(q, k, v, layout, sm_scale, is_causal)


attention.register_fake(_fake)


@torch.library.custom_op("cdna4_sage::attention_masked", mutates_args=())
def attention_masked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask: torch.Tensor, layout: str,
                     sm_scale: float, is_causal: bool) -> torch.Tensor:
    """attention with an attn_mask as torch SDPA takes it (bool True = attend, or additive of q's dtype; broadcastable
    to [B, H, q_len, kv_len]); no counterpart in the reference, which sends masked calls to SDPA.  Returns
    (B, Sq, H, D) contiguous."""
    return _attention.attention(q, k, v, layout, sm_scale if sm_scale > 0 else None, is_causal, attn_mask=attn_mask)


@attention_masked.register_fake
def _fake_masked(q, k, v, attn_mask, layout, sm_scale, is_causal):
    return _fake(q, k, v, layout, sm_scale, is_causal)
