// Packed variable-length attention (sageattn_varlen) without a host round trip.
//
// The reference loops over the sequences on the host after reading cu_seqlens back (src/sageattention/core.py:80-88)
// and makes one sageattn call per sequence.  Here the tables that describe the packed batch are built on the GPU
// from cu_seqlens, and five stream-ordered launches cover every sequence:
//   varlen_meta_kernel  (1 workgroup)  checks cu_seqlens, prefix sums of the padded key counts (kp), sequence
//                                      order for the attention (most keys first: long tiles start early), prefix
//                                      sums of the query tiles in that order (tpre)
//   varlen_prep_kernel                 tile table (sequence, head, query tile) per attention workgroup, owner of
//                                      each padded 128-key block (ktab), VS cleared
//   quant_varlen_kernel, quant_v_varlen_kernel, attn_kernel<..., VARLEN>   (sage_quant.hip, sage_attn.hip)
// Each sequence's quantization (per-token Q scales, 32-key K blocks counted from the sequence's first key, V
// channel maxima over the sequence) and attention (bottom-right causal per sequence) are those of a separate call.
// Invalid cu_seqlens (decreasing, negative, or past the packed totals) leave every table empty: no launch after the
// meta kernel touches memory outside the workspace and vs, the output is left as it was, and word 0 of the
// workspace reads 1.
#include <algorithm>

#include "sage_common.h"
#include "sage_host.h"

namespace sage {

int varlen_quant_impl(const void* q, int64_t qss, int64_t qsh, const void* k, int64_t kss, int64_t ksh, const void* v,
                      int64_t vss, int64_t vsh, int H, int Hkv, int TQ, int TKP, int D, int dtype, float qs_mul,
                      const int* cu_k, const int* kp, const int* ktab, int8_t* q8, float* qs, int8_t* k8, float* ks,
                      uint8_t* v8t, float* vs, void* stream);
int attn_varlen_impl(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                     const float* vs, void* out, int64_t oss, int64_t osh, int H, int Hkv, int TQ, int TKP, int D,
                     int causal, int out_dtype, int n_blocks, const void* tiles, const int* cu_q, const int* cu_k,
                     const int* kp, void* stream);

constexpr int VL_META_THREADS = 1024;
constexpr int VL_SORT_BINS = 2048;  // sequences ordered by min(ceil(kv_len / 64), 2047), descending

// Workspace layout (byte offsets, each region 256-byte aligned).
struct VarlenLayout {
  int64_t hdr, kp, order, tpre, ktab, tiles, bytes;
  int tkp;       // padded packed key rows per kv head
  int q_tiles;   // upper bound of the query tiles per head over all sequences
  int n_blocks;  // attention workgroups = H * q_tiles
};

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// sum_b pad128(len_b) <= total + 127 * batch and sum_b ceil(len_b / 128) <= (total + 127 * batch) / 128
static int varlen_layout(int batch, int H, int Hkv, int total_q, int total_k, VarlenLayout* L) {
  SAGE_REQUIRE(batch > 0 && H > 0 && Hkv > 0 && total_q > 0 && total_k > 0,
               "sage_forward_varlen: sizes must be positive (batch=%d H=%d Hkv=%d total_q=%d total_k=%d)", batch, H,
               Hkv, total_q, total_k);
  SAGE_REQUIRE(H % Hkv == 0, "sage_forward_varlen: heads %d not a multiple of kv heads %d", H, Hkv);
  const int64_t tkp = ((int64_t)total_k + 127ll * batch) / 128 * 128;
  const int64_t qt = ((int64_t)total_q + 127ll * batch) / 128;
  SAGE_REQUIRE(tkp * 128 < (1ll << 31) && (int64_t)H * qt < (1ll << 31),
               "sage_forward_varlen: packed batch too large (total_k=%d total_q=%d batch=%d)", total_k, total_q, batch);
  L->tkp = (int)tkp;
  L->q_tiles = (int)qt;
  L->n_blocks = (int)(H * qt);
  int64_t o = 0;
  L->hdr = o;
  o = align256(o + 64 * 4);
  L->kp = o;
  o = align256(o + (int64_t)(batch + 1) * 4);
  L->order = o;
  o = align256(o + (int64_t)batch * 4);
  L->tpre = o;
  o = align256(o + (int64_t)(batch + 1) * 4);
  L->ktab = o;
  o = align256(o + tkp / 128 * 4);
  L->tiles = o;
  o = align256(o + (int64_t)L->n_blocks * 16);
  L->bytes = o;
  return SAGE_OK;
}

// Inclusive scan of one int per thread over the workgroup (Hillis-Steele in LDS).
__device__ int block_inclusive_scan(int x, int* buf) {
  const int t = threadIdx.x;
  buf[t] = x;
  __syncthreads();
  for (int off = 1; off < VL_META_THREADS; off <<= 1) {
    const int y = t >= off ? buf[t - off] : 0;
    __syncthreads();
    buf[t] += y;
    __syncthreads();
  }
  const int r = buf[t];
  __syncthreads();
  return r;
}

__device__ __forceinline__ int pad128(int n) { return (n + 127) / 128 * 128; }

__global__ __launch_bounds__(VL_META_THREADS) void varlen_meta_kernel(const int* __restrict__ cu_q,
                                                                       const int* __restrict__ cu_k, int batch, int H,
                                                                       int total_q, int total_k, int* __restrict__ hdr,
                                                                       int* __restrict__ kp, int* __restrict__ order,
                                                                       int* __restrict__ tpre) {
  __shared__ int buf[VL_META_THREADS];
  __shared__ int bins[VL_SORT_BINS];
  __shared__ int bad;
  const int t = threadIdx.x;
  const int seg = (batch + VL_META_THREADS - 1) / VL_META_THREADS;
  const int lo = min(batch, t * seg), hi = min(batch, lo + seg);
  if (t == 0) bad = 0;
  for (int i = t; i < VL_SORT_BINS; i += VL_META_THREADS) bins[i] = 0;
  __syncthreads();

  // ---- validation and padded key counts ----
  int sk = 0;
  for (int b = lo; b < hi; ++b) {
    const int q0 = cu_q[b], q1 = cu_q[b + 1], k0 = cu_k[b], k1 = cu_k[b + 1];
    if (q0 < 0 || q1 < q0 || q1 > total_q || k0 < 0 || k1 < k0 || k1 > total_k) bad = 1;
    sk += pad128(k1 - k0);
  }
  __syncthreads();
  if (bad) {  // uniform: every table stays empty
    if (t == 0) {
      hdr[0] = 1;
      hdr[1] = 0;
      hdr[2] = 0;
    }
    return;
  }
  // ---- kp: exclusive prefix of the padded key counts, in batch order ----
  int run = block_inclusive_scan(sk, buf) - sk;
  for (int b = lo; b < hi; ++b) {
    kp[b] = run;
    run += pad128(cu_k[b + 1] - cu_k[b]);
  }
  if (t == VL_META_THREADS - 1) kp[batch] = run;  // the last thread's running sum is the total

  // ---- order: counting sort by key tiles, descending (positions inside a bin follow LDS atomics) ----
  for (int b = lo; b < hi; ++b) {
    const int key = min((cu_k[b + 1] - cu_k[b] + 63) / 64, VL_SORT_BINS - 1);
    atomicAdd(&bins[VL_SORT_BINS - 1 - key], 1);
  }
  __syncthreads();
  {
    constexpr int BPT = VL_SORT_BINS / VL_META_THREADS;
    int c[BPT], s = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      c[i] = bins[t * BPT + i];
      s += c[i];
    }
    int base = block_inclusive_scan(s, buf) - s;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      bins[t * BPT + i] = base;
      base += c[i];
    }
  }
  __syncthreads();
  for (int b = lo; b < hi; ++b) {
    const int key = min((cu_k[b + 1] - cu_k[b] + 63) / 64, VL_SORT_BINS - 1);
    order[atomicAdd(&bins[VL_SORT_BINS - 1 - key], 1)] = b;
  }
  __syncthreads();  // order[] (global, written by this workgroup) is visible to the workgroup after the barrier

  // ---- tpre: exclusive prefix of H * query tiles over the sorted order ----
  int st = 0;
  for (int i = lo; i < hi; ++i) {
    const int b = order[i];
    st += H * ((cu_q[b + 1] - cu_q[b] + 127) / 128);
  }
  run = block_inclusive_scan(st, buf) - st;
  for (int i = lo; i < hi; ++i) {
    tpre[i] = run;
    const int b = order[i];
    run += H * ((cu_q[b + 1] - cu_q[b] + 127) / 128);
  }
  if (t == VL_META_THREADS - 1) {
    tpre[batch] = run;
    hdr[0] = 0;
    hdr[1] = run;
    hdr[2] = kp[batch];
  }
}

// grid-stride over max(n_tiles, n_kblk, n_vs)
__global__ __launch_bounds__(256) void varlen_prep_kernel(const int* __restrict__ hdr, const int* __restrict__ cu_q,
                                                          const int* __restrict__ kp, const int* __restrict__ order,
                                                          const int* __restrict__ tpre, int batch, int H,
                                                          int causal, int n_tiles, int n_kblk, int4* __restrict__ tiles,
                                                          int* __restrict__ ktab, float* __restrict__ vs,
                                                          int64_t n_vs) {
  const int T = hdr[1], kp_total = hdr[2];
  const int64_t n = max((int64_t)max(n_tiles, n_kblk), n_vs);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    if (i < n_tiles) {
      int4 e = make_int4(-1, 0, 0, 0);
      if (i < T) {
        // last sorted position p with tpre[p] <= i (its sequence has tiles: tpre[p + 1] > i)
        int lo = 0, hi = batch - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (tpre[mid] <= i) lo = mid;
          else hi = mid - 1;
        }
        const int b = order[lo];
        const int r = (int)i - tpre[lo];
        const int nq = (cu_q[b + 1] - cu_q[b] + 127) / 128;
        // causal: the sequence's tiles longest first across its heads (its last query tile of every head, then the one
        // before, ...), so that its short tiles come last; otherwise head by head
        e = causal ? make_int4(b, r % H, nq - 1 - r / H, 0) : make_int4(b, r / nq, r % nq, 0);
      }
      tiles[i] = e;
    }
    if (i < n_kblk) {
      int owner = -1;
      const int x = (int)i * 128;
      if (x < kp_total) {
        int lo = 0, hi = batch - 1;  // last b with kp[b] <= x
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (kp[mid] <= x) lo = mid;
          else hi = mid - 1;
        }
        owner = lo;
      }
      ktab[i] = owner;
    }
    if (i < n_vs) vs[i] = 0.0f;
  }
}

static int check_packed(const void* p, int64_t ss, int64_t sh, const char* name) {
  SAGE_REQUIRE(p != nullptr, "sage_forward_varlen: %s is NULL", name);
  SAGE_REQUIRE(aligned16(p), "sage_forward_varlen: %s is not 16-byte aligned", name);
  SAGE_REQUIRE(ss % 8 == 0 && sh % 8 == 0 && ss >= 0 && sh >= 0,
               "sage_forward_varlen: %s strides (%lld, %lld) must be non-negative multiples of 8 elements", name,
               (long long)ss, (long long)sh);
  return SAGE_OK;
}

}  // namespace sage

extern "C" {

int sage_varlen_layout(int batch, int H, int Hkv, int total_q, int total_k, int* kv_rows, int64_t* workspace_bytes) {
  sage::clear_error();
  sage::VarlenLayout L;
  int rc = sage::varlen_layout(batch, H, Hkv, total_q, total_k, &L);
  if (rc) return rc;
  if (kv_rows) *kv_rows = L.tkp;
  if (workspace_bytes) *workspace_bytes = L.bytes;
  return SAGE_OK;
}

int sage_forward_varlen(const void* q, int64_t qss, int64_t qsh, const void* k, int64_t kss, int64_t ksh,
                        const void* v, int64_t vss, int64_t vsh, void* out, int64_t oss, int64_t osh,
                        const int* cu_seqlens_q, const int* cu_seqlens_k, int batch, int H, int Hkv, int total_q,
                        int total_k, int D, int dtype, int causal, float qs_mul, int8_t* q8, float* qs, int8_t* k8,
                        float* ks, uint8_t* v8t, float* vs, void* workspace, int64_t workspace_bytes, void* stream) {
  sage::clear_error();
  sage::VarlenLayout L;
  int rc = sage::varlen_layout(batch, H, Hkv, total_q, total_k, &L);
  if (rc) return rc;
  if (!sage::head_dim_ok(D))
    return sage::fail(SAGE_ERR_UNSUPPORTED, "sage_forward_varlen: head_dim %d (supported 64, 96, 128, 256)", D);
  if (dtype != SAGE_DTYPE_BF16 && dtype != SAGE_DTYPE_F16)
    return sage::fail(SAGE_ERR_UNSUPPORTED, "sage_forward_varlen: dtype code %d (bf16=0, f16=1)", dtype);
  if ((rc = sage::check_packed(q, qss, qsh, "q"))) return rc;
  if ((rc = sage::check_packed(k, kss, ksh, "k"))) return rc;
  if ((rc = sage::check_packed(v, vss, vsh, "v"))) return rc;
  if ((rc = sage::check_packed(out, oss, osh, "out"))) return rc;
  if ((rc = sage::check_qs_mul(qs_mul, "sage_forward_varlen"))) return rc;
  SAGE_REQUIRE(cu_seqlens_q && cu_seqlens_k, "sage_forward_varlen: cu_seqlens is NULL");
  SAGE_REQUIRE(q8 && qs && k8 && ks && v8t && vs, "sage_forward_varlen: an intermediate pointer is NULL");
  SAGE_REQUIRE(sage::aligned16(q8) && sage::aligned16(k8) && sage::aligned16(v8t) && sage::aligned16(vs),
               "sage_forward_varlen: q8 / k8 / v8t / vs must be 16-byte aligned");
  SAGE_REQUIRE(workspace != nullptr && workspace_bytes >= L.bytes,
               "sage_forward_varlen: workspace of %lld bytes, the layout needs %lld", (long long)workspace_bytes,
               (long long)L.bytes);
  SAGE_REQUIRE(((uintptr_t)workspace & 255u) == 0, "sage_forward_varlen: workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(workspace);
  int* hdr = reinterpret_cast<int*>(ws + L.hdr);
  int* kp = reinterpret_cast<int*>(ws + L.kp);
  int* order = reinterpret_cast<int*>(ws + L.order);
  int* tpre = reinterpret_cast<int*>(ws + L.tpre);
  int* ktab = reinterpret_cast<int*>(ws + L.ktab);
  int4* tiles = reinterpret_cast<int4*>(ws + L.tiles);
  hipStream_t st = (hipStream_t)stream;

  hipLaunchKernelGGL(sage::varlen_meta_kernel, dim3(1), dim3(sage::VL_META_THREADS), 0, st, cu_seqlens_q,
                     cu_seqlens_k, batch, H, total_q, total_k, hdr, kp, order, tpre);
  if ((rc = sage::check_launch("varlen meta launch"))) return rc;
  const int n_kblk = L.tkp / 128;
  const int64_t n_vs = (int64_t)batch * Hkv * sage::layout_dim(D);
  const int64_t n_items = std::max<int64_t>(std::max(L.n_blocks, n_kblk), n_vs);
  const int grid = (int)std::min<int64_t>((n_items + 255) / 256, 4096);
  hipLaunchKernelGGL(sage::varlen_prep_kernel, dim3(grid), dim3(256), 0, st, hdr, cu_seqlens_q, kp, order, tpre, batch,
                     H, causal ? 1 : 0, L.n_blocks, n_kblk, tiles, ktab, vs, n_vs);
  if ((rc = sage::check_launch("varlen prep launch"))) return rc;
  if ((rc = sage::varlen_quant_impl(q, qss, qsh, k, kss, ksh, v, vss, vsh, H, Hkv, total_q, L.tkp, D, dtype, qs_mul,
                                    cu_seqlens_k, kp, ktab, q8, qs, k8, ks, v8t, vs, stream)))
    return rc;
  return sage::attn_varlen_impl(q8, qs, k8, ks, v8t, vs, out, oss, osh, H, Hkv, total_q, L.tkp, D, causal, dtype,
                                L.n_blocks, tiles, cu_seqlens_q, cu_seqlens_k, kp, stream);
}

}  // extern "C"
