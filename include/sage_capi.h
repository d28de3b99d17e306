/*
 * libsage_capi: C ABI of the MI355X (gfx950) SageAttention path.
 *
 * This library replaces the reference's native launch boundary: rdna4_sage loads ahead-of-time code objects and
 * launches them with hipModuleLaunchKernel and a packed kernarg block per manifest entry
 * (src/rdna4_sage/_hip.py:52-73, kernel_build/build_kernels.py:34-37).  Here each of those launches is a typed C
 * entry point that takes plain device pointers, sizes and element strides, validates them on the host and launches
 * hipcc-built gfx950 kernels on the caller's stream.  Arguments are passed by value (no shared packing buffer), so
 * entry points are reentrant; nothing synchronises.
 *
 * Conventions
 *  - Return value: SAGE_OK (0) or a SAGE_ERR_* code; sage_last_error() gives the message (thread-local).  Every
 *    entry point checks all of its arguments before its first launch: a call rejected with SAGE_ERR_INVALID or
 *    SAGE_ERR_UNSUPPORTED has launched nothing and written no memory.
 *  - Memory: the caller owns every buffer (inputs, outputs, intermediates) and the library allocates nothing at run
 *    time; its only device memory is the static scratch array of sage_forward_noalloc (one per GPU it runs on).
 *  - Streams: `stream` is a hipStream_t (NULL = the default stream).
 *  - Element strides: (batch, seq, head) strides in elements; the head_dim axis must be contiguous; input base
 *    pointers 16-byte aligned and strides multiples of 8 elements (the quantizers load 16-byte vectors).
 *  - dtype: SAGE_DTYPE_BF16 or SAGE_DTYPE_F16; head_dim D = 64, 96, 128 or 256 (kernel_build/build_kernels.py:26).
 *    Q and K are rotated by the unnormalised Hadamard matrix of RB = min(D, 128) channels (block-diagonal for 256);
 *    D = 96 is not rotated (kernel_build/build_kernels.py:40-41, :102-104; sage_quant.py:18-30).
 *
 * Intermediate layouts (device memory, all contiguous; DL = sage_layout_dim(D): D, or 128 for D = 96 whose rows are
 * zero-padded; the attention kernel reads them as 128-channel tiles):
 *  - Q8  int8  [B, H, Sq, DL]             (head-major; the reference writes [B, Sq, H, D])
 *  - QS  fp32  [B, H, Sq]                 per-token scale / RB (D = 96: the scale itself), times the sm_scale fold
 *  - K8  int8  [B, Hkv, Skp, DL]          Skp = sage_kv_pad(Skv); rows >= Skv are zero
 *  - KS  fp32  [B, Hkv, Skp / 32]         one scale per 32 keys (not divided by RB)
 *  - V8T e4m3  [B, Hkv, DL, Skp]          V * 448 / amax, transposed; inside every 64-key group key 8g + 4h + r is
 *                                         stored at position 32h + 4g + r (the order the attention kernel's fp8 MFMA
 *                                         operand wants); keys >= Skv are zero
 *  - VS  fp32  [B, Hkv, DL]               per-channel max |v| over the sequence (0 for padding channels)
 *
 * Workspace: sage_attn_fwd / sage_forward may split the key range of the query tiles of a short last round over
 * several workgroups (a plan that depends on the problem shape and the device's CU count, see sage_attn_plan); the
 * partial softmax state of those tiles lives in a caller-provided workspace, 256-byte aligned.  Passing NULL runs
 * every tile whole (same results up to float rounding of the merge, lower throughput when the last round is short).
 */
#ifndef SAGE_CAPI_H
#define SAGE_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAGE_OK 0
#define SAGE_ERR_INVALID 1     /* bad pointer, size, stride or alignment */
#define SAGE_ERR_UNSUPPORTED 2 /* head_dim / dtype / causal shape the kernels are not built for */
#define SAGE_ERR_HIP 3         /* a HIP runtime call failed */

#define SAGE_DTYPE_BF16 0
#define SAGE_DTYPE_F16 1
#define SAGE_DTYPE_BOOL 2 /* attention masks only */

#define SAGE_KV_BLOCK 32  /* keys per K scale (kernel_build/build_kernels.py:30) */
#define SAGE_KV_PAD 128   /* K8 / V8T rows are padded to a multiple of this */

/* ABI version of this header (bumped on any signature change). */
int sage_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* sage_last_error(void);

/* Padded KV length Skp used by K8 / KS / V8T. */
int sage_kv_pad(int skv);

/* Channels DL of the Q8 / K8 / V8T / VS layouts for head_dim D (D, or 128 for D = 96); 0 if D is not supported.
   No counterpart in the reference (its Triton quantizers write D channels). */
int sage_layout_dim(int head_dim);

/* JSON description of the built kernels (architecture, head dims, tiles); static storage. */
const char* sage_manifest_json(void);

/*
 * Hadamard-rotate Q over head_dim and quantize to int8 with one scale per token.
 * Replaces the quant_q launch of src/rdna4_sage/_attention.py:125-126 (kernel kernel_build/sage_quant.py:33-48,
 * kernarg "<4Q5i4x2Q", build_kernels.py:36) and folds the sm_scale multiply of _attention.py:130-131:
 * QS = fp32(fp32(s / D) * qs_mul); pass qs_mul = 1.0f for the default scale.  qs_mul must be positive and finite
 * (SAGE_ERR_INVALID otherwise); the same holds for the qs_mul of every forward entry point.
 * q: [B, Sq, H, D] addressed as q + b*sb + s*ss + h*sh.
 */
int sage_quant_q(const void* q, int64_t sb, int64_t ss, int64_t sh, int B, int H, int Sq, int D, int dtype,
                 float qs_mul, int8_t* q8, float* qs, void* stream);

/*
 * Per-channel max |v| over the sequence, fp32 [B, Hkv, D].  Replaces
 * torch.linalg.vector_norm(v, ord=inf, dim=seq, dtype=float32) of src/rdna4_sage/_attention.py:120-121.
 * vs is overwritten (the library clears it with a fill kernel first).
 */
int sage_v_amax(const void* v, int64_t sb, int64_t ss, int64_t sh, int B, int Hkv, int Skv, int D, int dtype,
                float* vs, void* stream);

/*
 * Hadamard-rotate K and quantize to int8 (one scale per 32 keys); quantize V to E4M3 with the per-channel scale
 * 448 / max(vs, 1e-30) and store it transposed.  Replaces the quant_kv launch of src/rdna4_sage/_attention.py:127-129
 * (kernel kernel_build/sage_quant.py:51-70, kernarg "<7Q9i4x2Q", build_kernels.py:37).
 */
int sage_quant_kv(const void* k, int64_t ksb, int64_t kss, int64_t ksh, const void* v, int64_t vsb, int64_t vss,
                  int64_t vsh, int B, int Hkv, int Skv, int D, int dtype, const float* vs, int8_t* k8, float* ks,
                  uint8_t* v8t, void* stream);

/*
 * Work plan of sage_attn_fwd on the current device: query tiles (128 rows of one batch and head, numbered
 * ((b * H + h) * ceil(Sq / 128) + tile)) below *n_full run whole; each later tile splits its key tiles of 64 keys into
 * *chunks contiguous ranges merged by a second kernel.  *workspace_bytes is the workspace the split needs (0 when
 * nothing is split).  Output pointers may be NULL.  No counterpart in the reference (its launch is one workgroup per
 * query tile, src/rdna4_sage/_attention.py:133-139).
 */
int sage_attn_plan(int B, int H, int Sq, int Skv, int D, int causal, int* n_full, int* chunks, int64_t* workspace_bytes);

/*
 * int8 QK^T / fp8 PV flash attention with the reference's online softmax (lazy rescale, threshold 8 in log2
 * units), causal (bottom-right aligned: query i sees keys j <= i + Skv - Sq; requires Sq <= Skv) and grouped-query
 * heads (H % Hkv == 0).
 * Replaces the attn launch of src/rdna4_sage/_attention.py:133-139 (kernarg "<4Q3i4x6Q2i", build_kernels.py:35).
 * out: out + b*osb + s*oss + h*osh (element strides, head_dim contiguous), dtype out_dtype.
 * lse: optional fp32 [B, H, Sq] (natural-log logsumexp of the quantized logits); pass NULL to skip.
 * workspace: NULL, or at least the sage_attn_plan bytes for this shape (see "Workspace" above).
 */
int sage_attn_fwd(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                  const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq,
                  int Skv, int D, int causal, int out_dtype, float* lse, void* workspace, int64_t workspace_bytes,
                  void* stream);

/*
 * Row logsumexp of (Q K^T) * sm_scale over the keys (natural log), fp32 [B, H, Sq], computed from the bf16 / fp16
 * inputs with 16-bit MFMAs and fp32 accumulation (the value `return_lse` returns).  sm_scale <= 0 means 1/sqrt(D).
 * Causal masks are bottom-right aligned and need Sq <= Skv.  q / k addressed like sage_quant_q / sage_quant_kv.
 * Replaces the fp32 torch matmul + logsumexp of src/sageattention/core.py:23-44 (`_lse`).
 */
int sage_lse_fwd(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                 int64_t ksh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal, float sm_scale,
                 float* lse, void* stream);

/* Workspace bytes sage_forward needs for this shape on the current device (attention split state + per-chunk V
   maxima).  No counterpart in the reference. */
int sage_forward_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int64_t* workspace_bytes);

/*
 * The whole path in one call, on one stream.  Replaces the body of src/rdna4_sage/_attention.py:97-140 below
 * check_supported.  Intermediates are caller-owned buffers with the layouts above.  With a workspace of
 * sage_forward_workspace bytes: one launch quantizes Q and takes per-chunk V maxima, one quantizes K and V, then the
 * attention (and the merge of split tiles).  With workspace NULL: V maxima by atomics (fill + v_amax), quant_q,
 * quant_kv, unsplit attention.  Both give the same intermediates bit for bit.
 */
int sage_forward(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                 int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out, int64_t osb, int64_t oss,
                 int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal, float qs_mul,
                 int8_t* q8, float* qs, int8_t* k8, float* ks, uint8_t* v8t, float* vs, void* workspace,
                 int64_t workspace_bytes, void* stream);

/*
 * Packed variable-length batches: the padded key rows per kv head (*kv_rows, for the K8 / KS / V8T buffers of
 * sage_forward_varlen) and the bytes of its table workspace, from the packed sizes alone.  Either output may be NULL.
 */
int sage_varlen_layout(int batch, int H, int Hkv, int total_q, int total_k, int* kv_rows, int64_t* workspace_bytes);

/*
 * Packed variable-length attention in one stream-ordered pass, without reading cu_seqlens back to the host.
 * Replaces the host loop of src/sageattention/core.py:66-89 (sageattn_varlen: cu_seqlens .tolist(), one sageattn
 * call per sequence).  q: [total_q] tokens of H heads at q + t*qss + h*qsh (D contiguous); k / v: [total_k] tokens
 * of Hkv heads; out: [total_q] tokens of H heads, dtype = input dtype.  cu_seqlens_q / cu_seqlens_k: device int32
 * [batch + 1]; sequence i is queries [cu_q[i], cu_q[i+1]) against keys [cu_k[i], cu_k[i+1]), quantized and attended
 * exactly as a sage_forward call on that sequence alone (causal: bottom-right per sequence; query rows that see no
 * key are written as 0).  Rows outside every sequence are not written.  Intermediates (caller-owned, R = *kv_rows
 * of sage_varlen_layout): q8 int8 [H][total_q][D], qs fp32 [H][total_q], k8 int8 [Hkv][R][D], ks fp32
 * [Hkv][R / 32], v8t E4M3 [Hkv][D][R], vs fp32 [batch][Hkv][D]; sequence i's keys sit at rows kp[i] (sum of the
 * earlier sequences' lengths rounded up to 128).  workspace: sage_varlen_layout bytes, 256-byte aligned.  cu_seqlens
 * that decrease or pass total_q / total_k leave the output unwritten and set the workspace's first int32 to 1.
 */
int sage_forward_varlen(const void* q, int64_t qss, int64_t qsh, const void* k, int64_t kss, int64_t ksh,
                        const void* v, int64_t vss, int64_t vsh, void* out, int64_t oss, int64_t osh,
                        const int* cu_seqlens_q, const int* cu_seqlens_k, int batch, int H, int Hkv, int total_q,
                        int total_k, int D, int dtype, int causal, float qs_mul, int8_t* q8, float* qs, int8_t* k8,
                        float* ks, uint8_t* v8t, float* vs, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Attention masks with torch SDPA's semantics: mask_dtype SAGE_DTYPE_BOOL (a nonzero byte = the query attends the
 * key) or an additive float mask of the inputs' dtype (SAGE_DTYPE_BF16 / SAGE_DTYPE_F16: added to the scaled scores,
 * -inf = masked).  The mask is addressed as mask + b*msb + h*msh + i*msq + j (in elements) for batch b, query head h,
 * query i, key j; the key axis is contiguous and a stride of 0 broadcasts that axis, as torch's expand gives.  No
 * counterpart in the reference: src/rdna4_sage/__init__.py:78-79 sends every masked call to torch SDPA
 * (`attn_mask is not None` -> `_sdpa`).
 *
 * sage_mask_workspace: bytes of the workspace sage_forward_masked needs for this shape and mask on the current device
 * (the attention's split state, the per-chunk V maxima and the mask's tables).
 */
int sage_mask_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int mask_dtype, int64_t msb,
                        int64_t msh, int64_t msq, int64_t* workspace_bytes);

/*
 * sage_forward with an attention mask: the same quantization and quantized attention, with the mask applied to the
 * scores (bool: masked keys at -inf; float: the values added, ANDed / combined with the bottom-right causal mask when
 * causal is set).  A query row that sees no key is written as 0 (as torch 2.10's SDPA writes it, on gfx950 and on the CPU).  Same arguments as
 * sage_forward plus the mask; workspace: sage_mask_workspace bytes, 256-byte aligned (required).  Replaces, for
 * these masks, the torch SDPA call of src/rdna4_sage/__init__.py:44-56 (`_sdpa`) that the reference makes for every
 * call with an attn_mask.
 */
int sage_forward_masked(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                        int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out, int64_t osb,
                        int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal,
                        float qs_mul, const void* mask, int mask_dtype, int64_t msb, int64_t msh, int64_t msq,
                        int8_t* q8, float* qs, int8_t* k8, float* ks, uint8_t* v8t, float* vs, void* workspace,
                        int64_t workspace_bytes, void* stream);

/*
 * sage_forward without any allocation: the intermediates (Q8, QS, K8, KS, V8T, VS) and the workspace live in the
 * library's own device array of SAGE_NOALLOC_SCRATCH_BYTES per GPU (each GPU the library runs on holds its copy until
 * the process ends); the caller passes only the inputs and the output, with sage_forward's meaning.  For callers
 * that cannot call hipMalloc or an allocating library (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it).  No counterpart in the reference.  A shape whose intermediates and workspace exceed the array
 * returns SAGE_ERR_INVALID (128 MiB holds e.g. [1, 24, 4608, 128], 69 MB, and [2, 32/8, 8192, 128], 103 MB).  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU (different streams or threads without
 * ordering) race and give wrong outputs without an error; calls ordered on one stream do not.  Nothing in the array
 * needs clearing between calls.  The first call on each GPU looks up the array's address (hipGetSymbolAddress, which
 * may load the code object): make one eager call per GPU before capturing calls into a HIP graph.
 */
#define SAGE_NOALLOC_SCRATCH_BYTES (128ll << 20)
int sage_forward_noalloc(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb,
                         int64_t kss, int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out,
                         int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype,
                         int causal, float qs_mul, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAGE_CAPI_H */
