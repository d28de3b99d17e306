"""The reference's import name, backed by the gfx950 implementation in cdna4_sage.

Callers written against crashingalexsan/RDNA4-SageAttention use ``import rdna4_sage`` and
``torch.ops.rdna4_sage.attention`` (src/rdna4_sage/__init__.py:17, src/rdna4_sage/ops.py:7); both resolve here to the
same kernels, routing and error behaviour as ``cdna4_sage``.  RDNA4_SAGE_MIN_WORK / RDNA4_SAGE_MIN_KV are honoured.
"""
from cdna4_sage import (ARCHS, HEAD_DIMS, MIN_KV, MIN_WORK, Unsupported, _plain_eager, _sdpa, _worth_it,
                        check_supported, device_arch, is_available, sageattn)
from cdna4_sage._attention import attention as _attention_impl

from . import ops

__all__ = ["sageattn", "attention", "is_available", "Unsupported", "ARCHS", "HEAD_DIMS"]
__version__ = "0.1.0"


def attention(q, k, v, tensor_layout="HND", sm_scale=None, is_causal=False):
    """Run the int8/fp8 kernel (through torch.ops.rdna4_sage.attention when traced, its implementation directly in
    eager mode); raises Unsupported if it cannot."""
    sm = float(sm_scale or 0.0)
    if not _plain_eager(q, k, v):
        out = ops.attention(q, k, v, tensor_layout, sm, bool(is_causal))
    else:
        out = _attention_impl(q, k, v, tensor_layout, sm if sm > 0 else None, bool(is_causal))
    return out.transpose(1, 2) if tensor_layout == "HND" else out
