"""SageAttention 2.2 API on top of cdna4_sage (AMD MI355X, gfx950).

Every public function of SageAttention 2.2 keeps its signature (reference: src/sageattention/core.py:47-129).  All of
them run the same path (Hadamard-rotated int8 Q K^T, fp8 P V with per-channel V scales); kernel-selection arguments
such as qk_quant_gran, pv_accum_dtype, smooth_k, smooth_v or value_dtype are accepted and ignored.  Calls the gfx950
kernels cannot run or would not win on (small problems, unsupported head dims or GPUs, masks of another dtype) use torch
SDPA, so the functions work on any device torch supports; bool and additive masks of the inputs' dtype run on the
kernels.
"""
from typing import Any, Optional

import torch

import cdna4_sage

_LSE_SCORE_BUDGET = 64 * 2**20  # fp32 scores per chunk of the LSE pass (~256 MB)


def _as_hnd(t: torch.Tensor, tensor_layout: str) -> torch.Tensor:
    if tensor_layout == "HND":
        return t
    if tensor_layout == "NHD":
        return t.transpose(1, 2)
    raise ValueError(f"tensor_layout must be 'HND' or 'NHD', got {tensor_layout!r}")


def _lse(q, k, tensor_layout, is_causal, sm_scale):
    """Row logsumexp of Q K^T * scale over the keys, fp32 [B, H, q_len], on the unquantized inputs
    (reference: src/sageattention/core.py:23-44).  Causal masks are bottom-right aligned.  On gfx950 the LSE kernel
    computes it (16-bit products exact in fp32, fp32 accumulation); elsewhere, and for shapes the kernel does not take,
    the query heads that share a kv head are processed together with one fp32 batched product per row chunk."""
    _as_hnd(q, tensor_layout)  # layout check (ValueError, as the reference)
    try:
        return cdna4_sage.lse(q, k, tensor_layout, sm_scale, is_causal)
    except cdna4_sage.Unsupported:
        pass
    q, k = _as_hnd(q, tensor_layout), _as_hnd(k, tensor_layout)
    B, H, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    if q.numel() == 0 or Hkv == 0:
        return torch.empty((B, H, Sq), device=q.device, dtype=torch.float32)   # no query rows: nothing to compute
    rep = H // Hkv
    scale = D ** -0.5 if sm_scale is None else sm_scale
    out = torch.empty((B, H, Sq), device=q.device, dtype=torch.float32)
    rows = max(1, _LSE_SCORE_BUDGET // max(1, Skv * rep))
    key_idx = torch.arange(Skv, device=q.device)
    for b in range(B):
        for g in range(Hkv):
            kt = k[b, g].float().t().contiguous()                       # [D, Skv]
            qg = q[b, g * rep:(g + 1) * rep]                             # [rep, Sq, D]
            for r0 in range(0, Sq, rows):
                r1 = min(Sq, r0 + rows)
                sc = torch.matmul(qg[:, r0:r1].float(), kt) * scale      # [rep, rows, Skv]
                if is_causal:
                    last = torch.arange(r0, r1, device=q.device) + (Skv - Sq)
                    sc.masked_fill_(key_idx[None, None, :] > last[None, :, None], float("-inf"))
                out[b, g * rep:(g + 1) * rep, r0:r1] = torch.logsumexp(sc, dim=-1)
    return out


def sageattn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    return_lse: bool = False,
    **kwargs: Any,
):
    """q / k / v of dtype fp16 or bf16, laid out "HND" [batch, heads, tokens, head_dim] or "NHD" [batch, tokens,
    heads, head_dim].  The result keeps that layout and dtype; return_lse=True adds the fp32 logsumexp of every query
    row, [batch, heads, q_len].  A causal mask aligns the last query with the last key.  attn_mask is read from the
    keyword arguments only (ComfyUI inspects this signature and expects no such parameter); bool masks and additive
    ones of the inputs' dtype run on the kernel.  The logsumexp ignores any mask, as the reference's does."""
    if (return_lse and q.is_cuda and not torch.compiler.is_compiling()
            and not torch.cuda.is_current_stream_capturing()):
        # the LSE pass does not depend on the attention: it runs on a side stream (default priority) concurrently with
        # the quantizers and the attention kernel on the caller's stream, which waits for it before returning (under
        # graph capture or tracing the two run one after the other on the caller's stream)
        cur = torch.cuda.current_stream(q.device)
        side = _side_stream(q.device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            lse = _lse(q, k, tensor_layout, is_causal, sm_scale)
        q.record_stream(side)
        k.record_stream(side)
        out = cdna4_sage.sageattn(q, k, v, tensor_layout=tensor_layout, is_causal=is_causal, sm_scale=sm_scale,
                                  attn_mask=kwargs.get("attn_mask"))
        cur.wait_stream(side)
        lse.record_stream(cur)
        return out, lse
    out = cdna4_sage.sageattn(q, k, v, tensor_layout=tensor_layout, is_causal=is_causal, sm_scale=sm_scale,
                              attn_mask=kwargs.get("attn_mask"))
    if return_lse:
        return out, _lse(q, k, tensor_layout, is_causal, sm_scale)
    return out


_side_streams = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _side_streams:
        _side_streams[idx] = torch.cuda.Stream(device=idx)
    return _side_streams[idx]


def sageattn_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    smooth_k: bool = True,
    **kwargs: Any,
) -> torch.Tensor:
    """Sequences packed along the token axis: q is [sum of query lengths, heads, head_dim], k and v
    [sum of key lengths, kv heads, head_dim]; cu_seqlens_q / cu_seqlens_k hold the batch + 1 sequence offsets.

    The reference reads the offsets back to the host and sends every sequence through sageattn on its own
    (src/sageattention/core.py:80-88), so each sequence takes sageattn's route: the quantized kernel when it is long
    enough (kv_len >= MIN_KV and heads * q_len * kv_len, halved when causal, >= MIN_WORK), torch SDPA otherwise.  This
    does the same: after reading the offsets, the sequences the kernel takes run in one packed stream-ordered pass of
    the int8/fp8 kernels (bit-equal, per sequence, to a call on that sequence with every query tile whole), and the
    others through sageattn one by one.  Under graph capture or torch.compile tracing, where the offsets cannot be
    read back, or with CDNA4_SAGE_VARLEN_ROUTE=0, the packed pass takes every sequence (no host synchronisation; the
    short ones are then quantized too).  Without a gfx950 GPU, or when the longest key sequence is below MIN_KV, every
    sequence goes through sageattn; empty query sequences are skipped."""
    try:
        mk = None if max_seqlen_k is None else int(max_seqlen_k)
    except (TypeError, ValueError):
        mk = None
    if q.is_cuda and (mk is None or mk >= cdna4_sage.MIN_KV):
        sync_free = (not cdna4_sage.VARLEN_ROUTE or torch.compiler.is_compiling()
                     or torch.cuda.is_current_stream_capturing())
        try:
            if sync_free:
                return cdna4_sage.attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                                   sm_scale=sm_scale, is_causal=is_causal)
            seqs = _sequences(cu_seqlens_q, cu_seqlens_k)
            fast = [_kernel_takes(q1 - q0, k1 - k0, q.shape[1], is_causal) for q0, q1, k0, k1 in seqs]
            if any(fast):
                out = cdna4_sage.attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                                  sm_scale=sm_scale, is_causal=is_causal)
                for (q0, q1, k0, k1), f in zip(seqs, fast):
                    if not f:
                        out[q0:q1] = _one_sequence(q, k, v, q0, q1, k0, k1, is_causal, sm_scale)
                return out
        except cdna4_sage.Unsupported:
            pass
    out = torch.empty_like(q)
    for q0, q1, k0, k1 in _sequences(cu_seqlens_q, cu_seqlens_k):
        out[q0:q1] = _one_sequence(q, k, v, q0, q1, k0, k1, is_causal, sm_scale)
    return out


def _sequences(cu_seqlens_q, cu_seqlens_k):
    """(q0, q1, k0, k1) of every sequence with at least one query, from offsets read back to the host."""
    bq = [int(x) for x in cu_seqlens_q.tolist()]
    bk = [int(x) for x in cu_seqlens_k.tolist()]
    return [(q0, q1, k0, k1) for (q0, q1), (k0, k1) in zip(zip(bq[:-1], bq[1:]), zip(bk[:-1], bk[1:])) if q1 > q0]


def _kernel_takes(sq, skv, heads, is_causal):
    """Whether sageattn on one sequence of a packed batch runs the kernel: the router's size rule (cdna4_sage._worth_it
    with batch 1) and the kernel's causal shapes (q_len <= kv_len)."""
    work = heads * sq * skv // (2 if is_causal else 1)
    return skv >= cdna4_sage.MIN_KV and work >= cdna4_sage.MIN_WORK and not (is_causal and sq > skv)


def _one_sequence(q, k, v, q0, q1, k0, k1, is_causal, sm_scale):
    return sageattn(q[q0:q1].unsqueeze(0), k[k0:k1].unsqueeze(0), v[k0:k1].unsqueeze(0), tensor_layout="NHD",
                    is_causal=is_causal, sm_scale=sm_scale)[0]


def _variant(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False, **kwargs):
    return sageattn(q, k, v, tensor_layout=tensor_layout, is_causal=is_causal, sm_scale=sm_scale,
                    return_lse=return_lse, attn_mask=kwargs.get("attn_mask"))


def sageattn_qk_int8_pv_fp16_triton(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                    quantization_backend: str = "triton", is_causal: bool = False,
                                    attn_mask: Optional[torch.Tensor] = None, sm_scale: Optional[float] = None,
                                    smooth_k: bool = True, return_lse: bool = False, **kwargs: Any):
    return _variant(q, k, v, tensor_layout, is_causal, sm_scale, return_lse, attn_mask=attn_mask)


def sageattn_qk_int8_pv_fp16_cuda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                  is_causal: bool = False, qk_quant_gran: str = "per_thread",
                                  sm_scale: Optional[float] = None, pv_accum_dtype: str = "fp32",
                                  smooth_k: bool = True, smooth_v: bool = False, return_lse: bool = False,
                                  **kwargs: Any):
    return _variant(q, k, v, tensor_layout, is_causal, sm_scale, return_lse)


def sageattn_qk_int8_pv_fp8_cuda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                 is_causal: bool = False, qk_quant_gran: str = "per_thread",
                                 sm_scale: Optional[float] = None, pv_accum_dtype: str = "fp32+fp16",
                                 smooth_k: bool = True, smooth_v: bool = False, return_lse: bool = False,
                                 **kwargs: Any):
    return _variant(q, k, v, tensor_layout, is_causal, sm_scale, return_lse)


def sageattn_qk_int8_pv_fp8_cuda_sm90(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                      is_causal: bool = False, qk_quant_gran: str = "per_thread",
                                      sm_scale: Optional[float] = None, pv_accum_dtype: str = "fp32+fp32",
                                      smooth_k: bool = True, return_lse: bool = False, **kwargs: Any):
    return _variant(q, k, v, tensor_layout, is_causal, sm_scale, return_lse)


def sageattn_qk_int8_pv_gfx12_native(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                     is_causal: bool = False, qk_quant_gran: str = "per_warp",
                                     sm_scale: Optional[float] = None, pv_accum_dtype: Optional[str] = None,
                                     value_dtype: str = "fp8", smooth_k: bool = True, smooth_v: bool = False,
                                     return_lse: bool = False, **kwargs: Any):
    return _variant(q, k, v, tensor_layout, is_causal, sm_scale, return_lse)
