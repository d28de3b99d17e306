"""SageAttention-style int8 QK / fp8 PV attention for AMD MI355X (gfx950, CDNA4).

Hand-written HIP kernels (Hadamard int8 quantizers, int8/fp8 MFMA flash attention) built ahead of time by hipcc into
libsage_capi.so and launched through its C ABI on torch's current stream.

    import cdna4_sage
    out = cdna4_sage.sageattn(q, k, v, tensor_layout="HND")   # drop-in for sageattention.sageattn

Routing mirrors the reference's src/rdna4_sage/__init__.py:20-84: small problems, unsupported shapes or GPUs, masks
of another dtype and causal calls with q_len > kv_len go to torch's SDPA binding; everything else runs the gfx950
kernels, including two cases the reference sends to SDPA: causal calls with q_len < kv_len (bottom-right aligned) and
attn_masks (bool, or additive of q's dtype; set CDNA4_SAGE_NATIVE_MASK=0 to send masks to SDPA as the reference
does).
attention_varlen runs packed variable-length batches in one pass.
"""
import os

import torch
from torch.nn.attention.bias import causal_lower_right

from . import ops
from ._attention import (ARCHS, HEAD_DIMS, Unsupported, attention_varlen, check_supported, device_arch, lse,
                         mask_view)
from ._attention import attention as _attention_impl

__all__ = ["sageattn", "attention", "attention_varlen", "lse", "is_available", "Unsupported", "ARCHS", "HEAD_DIMS"]
__version__ = "0.1.0"

# Fallbacks call torch's C entry point of SDPA directly: a caller may have monkey-patched
# F.scaled_dot_product_attention to point at sageattn, and the Python-level function would then lead straight back
# here (reference CHANGELOG 2.2.0+rdna4.0.2.1).
_torch_sdpa = torch._C._nn.scaled_dot_product_attention


def _env_int(names, default):
    for n in names:
        if os.environ.get(n):
            return int(os.environ[n])
    return default


# Size thresholds of the kernel route: below them the quantization pass and launches cost more than the int8 / fp8
# products save, and SDPA runs.  CDNA4_SAGE_* override; the reference's RDNA4_SAGE_* names are read as well.
MIN_WORK = _env_int(("CDNA4_SAGE_MIN_WORK", "RDNA4_SAGE_MIN_WORK"), 64 * 2**20)  # batch * heads * q_len * kv_len
MIN_KV = _env_int(("CDNA4_SAGE_MIN_KV", "RDNA4_SAGE_MIN_KV"), 1024)
# attn_masks (bool, or additive of q's dtype) run on the kernel (quantized like every other call); 0 restores the
# reference's SDPA routing.
NATIVE_MASK = _env_int(("CDNA4_SAGE_NATIVE_MASK",), 1) != 0
# sageattention.sageattn_varlen routes every sequence of a packed batch as the reference does (offsets read back, the
# short sequences to SDPA); 0 runs one quantized pass over every sequence without reading the offsets back.
VARLEN_ROUTE = _env_int(("CDNA4_SAGE_VARLEN_ROUTE",), 1) != 0


def is_available(device=None) -> bool:
    """True when the current (or given) GPU is gfx950, the only architecture the kernels are built for."""
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index or 0)
    return device_arch(dev) in ARCHS


def _plain_eager(*ts) -> bool:
    """True for an eager call on plain tensors: no torch.compile / export tracing, no tensor subclass (fake or
    functional tensors), no active dispatch mode (make_fx and the like) and no autograd recording on the inputs.  Such
    calls may run the op's implementation directly; anything else goes through the registered op, so that tracers see
    its fake implementation and autograd sees an op without a derivative (backward raises, as in the reference)."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack() > 0:
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in ts):
        return False
    return all(type(t) is torch.Tensor for t in ts)


def attention(q, k, v, tensor_layout="HND", sm_scale=None, is_causal=False, attn_mask=None):
    """Run the int8/fp8 kernel; raises Unsupported if it cannot.  Output in the input layout and dtype.
    Causal attention is bottom-right aligned and needs q_len <= kv_len.  attn_mask: None, a boolean mask (True =
    attend) or an additive mask of q's dtype, broadcastable to [B, H, q_len, kv_len] as torch SDPA takes it; a query
    row that sees no key is 0."""
    sm = float(sm_scale or 0.0)
    if not _plain_eager(q, k, v):  # traced: the registered op, which tracers see through its fake impl
        if attn_mask is None:
            out = ops.attention(q, k, v, tensor_layout, sm, bool(is_causal))
        else:
            out = ops.attention_masked(q, k, v, attn_mask, tensor_layout, sm, bool(is_causal))
    else:  # eager: the op's implementation itself, without the dispatcher's ~20 us per call
        out = _attention_impl(q, k, v, tensor_layout, sm if sm > 0 else None, bool(is_causal), attn_mask=attn_mask)
    return out.transpose(1, 2) if tensor_layout == "HND" else out


def _sdpa(q, k, v, tensor_layout, is_causal, sm_scale, attn_mask):
    if q.numel() == 0:
        # no query rows (empty batch, no heads or no tokens): the empty output itself.  torch SDPA raises for an
        # empty batch on the GPU and stops the process with SIGFPE for zero heads (torch 2.10, CPU and gfx950).
        return q.new_empty(tuple(q.shape[:-1]) + (v.shape[-1],))
    if tensor_layout == "NHD":
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    gqa = q.shape[1] != k.shape[1]
    Sq, Skv = q.shape[2], k.shape[2]
    if is_causal and (Sq != Skv or attn_mask is not None):
        # with q_len != kv_len (or a mask to combine) the causal triangle is anchored at the last key, the convention
        # SageAttention and FlashAttention use, which SDPA's is_causal flag does not follow
        causal = causal_lower_right(Sq, Skv)._materialize(q.device)
        if attn_mask is None:
            attn_mask = causal
        else:
            attn_mask = (attn_mask.masked_fill(~causal, float("-inf")) if attn_mask.dtype != torch.bool
                         else attn_mask & causal)
        is_causal = False
    out = _torch_sdpa(q, k, v, attn_mask=attn_mask, is_causal=is_causal, scale=sm_scale, enable_gqa=gqa)
    return out.transpose(1, 2) if tensor_layout == "NHD" else out


def _worth_it(q, k, tensor_layout, is_causal=False):
    if tensor_layout == "HND":
        B, H, Sq, _ = q.shape
        Skv = k.shape[2]
    else:
        B, Sq, H, _ = q.shape
        Skv = k.shape[1]
    work = B * H * Sq * Skv // (2 if is_causal else 1)
    return Skv >= MIN_KV and work >= MIN_WORK


def sageattn(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, attn_mask=None, return_lse=False, **kwargs):
    """Drop-in for sageattention.sageattn.  Uses the gfx950 kernel when it applies and pays off, torch SDPA otherwise
    (masks of another dtype, causal with q_len > kv_len, unsupported shapes or GPUs, small problems).  Causal attention
    is bottom-right aligned as in SageAttention / FlashAttention.  A bool attn_mask, or an additive one of q's dtype,
    runs on the kernel (a query row that sees no key gives 0 there, as torch SDPA gives).  Extra SageAttention kwargs are
    ignored."""
    if return_lse:
        raise NotImplementedError("cdna4_sage: return_lse is not supported here; use sageattention.sageattn")
    if (attn_mask is not None and not NATIVE_MASK) or not _worth_it(q, k, tensor_layout, is_causal):
        return _sdpa(q, k, v, tensor_layout, is_causal, sm_scale, attn_mask)
    try:
        check_supported(q, k, v, tensor_layout, is_causal)
        if attn_mask is not None:
            mask_view(attn_mask, q, k, tensor_layout)
    except Unsupported:
        return _sdpa(q, k, v, tensor_layout, is_causal, sm_scale, attn_mask)
    return attention(q, k, v, tensor_layout, sm_scale, is_causal, attn_mask=attn_mask)
