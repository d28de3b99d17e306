// Boolean attention masks (torch SDPA's bool attn_mask, True = attend): the bit and class tables that the mask
// variant of attn_kernel reads, and the one-call masked forward.
//
// The reference has no masked kernel: src/rdna4_sage/__init__.py:78-79 sends every call with an attn_mask to torch
// SDPA.  Here the mask is turned, on the GPU and in the call's stream, into
//   bits  one 32-bit word per (mask row, 64-key tile, lane half hf) in the order of the attention kernel's QK
//         accumulator (bit 16 kb + v <-> key 64 t + 32 kb + 8 (v / 4) + 4 hf + v % 4), so the kernel masks a score
//         with one bit extract and one bit select;
//   cls   one entry per (32-row group, tile): 0 = no row sees a key of the tile (the wave skips it), 1 = every row
//         sees every key (the mask-free tile body), 2 = mixed (the bit-masked body);
//   range one (first, last + 1) tile pair per 128-row block (an attention workgroup's rows): the tiles outside it
//         are not visited at all.
// Keys past kv_len and, with the causal flag, keys past the bottom-right diagonal are folded into the bits.
#include "sage_common.h"
#include "sage_host.h"

namespace sage {

int forward_quant_impl(const void*, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, int64_t, const void*,
                       int64_t, int64_t, int64_t, int, int, int, int, int, int, int, float, int8_t*, float*, float*,
                       int8_t*, float*, uint8_t*, float*, void*);
int64_t vamax_partial_bytes(int B, int Hkv, int Skv, int D);
int attn_mask_plan_impl(int B, int H, int Sq, int Skv, int D, int64_t* ws);
int attn_mask_impl(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                   const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq,
                   int Skv, int D, int out_dtype, const MaskTabs* mt, void* workspace, void* stream);

// Extents of the tables.  A mask axis with stride 0 (broadcast) is stored once; rows are stored when the mask has a
// row axis or the causal flag makes rows differ.
struct MaskShape {
  int mb, mh, mq, mg, nt, nrb;
  int64_t bits_words, cls_entries, range_entries;
};

static MaskShape mask_shape(int B, int H, int Sq, int Skv, int64_t msb, int64_t msh, int64_t msq, int causal) {
  MaskShape m;
  m.mb = msb == 0 ? 1 : B;
  m.mh = msh == 0 ? 1 : H;
  const bool rows = msq != 0 || causal;
  m.mq = rows ? Sq : 1;
  m.mg = rows ? (Sq + 31) / 32 : 1;
  m.nrb = rows ? (Sq + 127) / 128 : 1;
  m.nt = (Skv + 63) / 64;
  m.bits_words = (int64_t)m.mb * m.mh * m.mq * m.nt * 2;
  m.cls_entries = (int64_t)m.mb * m.mh * m.mg * m.nt;
  m.range_entries = (int64_t)m.mb * m.mh * m.nrb;
  return m;
}

static int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// Workspace of sage_forward_masked: the attention plan's split state, the per-chunk V maxima, the bits, the classes,
// the ranges (each 256-byte aligned).
struct MaskWorkspace {
  int64_t attn, vpart, bits, cls, range, total;
};

static int mask_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, const MaskShape& m, MaskWorkspace* w) {
  int rc = attn_mask_plan_impl(B, H, Sq, Skv, D, &w->attn);
  if (rc) return rc;
  w->vpart = align256(w->attn);
  w->bits = w->vpart + align256(vamax_partial_bytes(B, Hkv, Skv, D));
  w->cls = w->bits + align256(m.bits_words * 4);
  w->range = w->cls + align256(m.cls_entries * 4);
  w->total = w->range + align256(m.range_entries * 8);
  return SAGE_OK;
}

// One wave per (mask batch-head, 32-row group, tile): lane (row r = lane % 32 of the group, half hf = lane / 32)
// builds its word from the 32 mask bytes of its keys (8 runs of 4 consecutive keys: run j holds keys
// 64 t + 8 j + 4 hf + i at bits 4 j + i); two ballots over the wave give the class.  Rows past q_len (and, for a
// mask without rows, every row but 0) count as neither seeing nor missing a key.  A4: mask rows start 4-byte
// aligned, so a run inside kv_len is one 32-bit load.  grid = mb * mh * mg * ceil(nt / 4) blocks of 256 threads.
template <bool A4>
__global__ __launch_bounds__(256) void mask_prep_kernel(const uint8_t* __restrict__ mask, int64_t msb, int64_t msh,
                                                        int64_t msq, int mh, int mq, int mg, int nt, int Sq, int Skv,
                                                        int causal, uint32_t* __restrict__ bits,
                                                        int* __restrict__ cls) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, hf = lane >> 5;
  const int ntb = (nt + 3) >> 2;
  const int t = (int)(blockIdx.x % ntb) * 4 + wave;
  const int rest = (int)(blockIdx.x / ntb);
  const int g = rest % mg;
  const int mbh = rest / mg;
  if (t >= nt) return;  // the whole wave
  const int mbi = mbh / mh, mhi = mbh % mh;
  const int q = g * 32 + r;  // table row (mq == 1: row 0 only)
  const bool real = mq == 1 ? r == 0 : q < Sq;
  uint32_t w = 0;
  if (real) {
    const uint8_t* row = mask + mbi * msb + mhi * msh + (int64_t)q * msq;
    const int lim = causal ? min(Skv - 1, q + (Skv - Sq)) : Skv - 1;  // last key the row may see
    const int k0 = t * 64 + 4 * hf;
    uint32_t b4[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kj = k0 + 8 * j;
      if (A4 && kj + 3 < Skv) {
        b4[j] = *reinterpret_cast<const uint32_t*>(row + kj);
      } else {
        b4[j] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kj + i < Skv) b4[j] |= (uint32_t)row[kj + i] << (8 * i);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool vis = ((b4[j] >> (8 * i)) & 0xFFu) != 0 && k0 + 8 * j + i <= lim;
        w |= (uint32_t)vis << (4 * j + i);
      }
    bits[(((int64_t)mbh * mq + q) * nt + t) * 2 + hf] = w;
  }
  const uint64_t any = __ballot(real && w != 0);
  const uint64_t all = __ballot(!real || w == 0xFFFFFFFFu);
  if (lane == 0) cls[((int64_t)mbh * mg + g) * nt + t] = any == 0 ? 0 : (all == ~0ull ? 1 : 2);
}

// One wave per (mask batch-head, 128-row block): the first and one past the last tile whose class is not 0 in any of
// the block's four 32-row groups (groups past the last one repeat it), (nt, 0) when there is none.  Lanes scan the
// 4 x nt classes with all their loads in flight, then a wave reduction.  grid = ceil(n / 4) blocks of 256 threads,
// n = mb * mh * nrb.
__global__ __launch_bounds__(256) void mask_range_kernel(const int* __restrict__ cls, int mg, int nt, int nrb, int n,
                                                         int2* __restrict__ range) {
  const int wid = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (wid >= n) return;  // the whole wave
  const int lane = threadIdx.x & 63;
  const int mbh = wid / nrb, rb = wid % nrb;
  int lo = nt, hi = -1;
  for (int i = lane; i < 4 * nt; i += 64) {
    const int g = min(rb * 4 + i / nt, mg - 1), t = i % nt;
    if (cls[((int64_t)mbh * mg + g) * nt + t] != 0) {
      lo = min(lo, t);
      hi = max(hi, t);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o));
    hi = max(hi, __shfl_xor(hi, o));
  }
  if (lane == 0) range[wid] = make_int2(lo, hi + 1);
}

static int launch_mask_prep(const void* mask, int64_t msb, int64_t msh, int64_t msq, int Sq, int Skv, int causal,
                            const MaskShape& m, uint32_t* bits, int* cls, int2* range, hipStream_t st) {
  const bool a4 = ((uintptr_t)mask & 3u) == 0 && msb % 4 == 0 && msh % 4 == 0 && msq % 4 == 0;
  const int64_t blocks = (int64_t)m.mb * m.mh * m.mg * ((m.nt + 3) / 4);
  const uint8_t* mp = static_cast<const uint8_t*>(mask);
  if (a4)
    hipLaunchKernelGGL(mask_prep_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st, mp, msb, msh, msq, m.mh, m.mq,
                       m.mg, m.nt, Sq, Skv, causal, bits, cls);
  else
    hipLaunchKernelGGL(mask_prep_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, mp, msb, msh, msq, m.mh,
                       m.mq, m.mg, m.nt, Sq, Skv, causal, bits, cls);
  const int n = (int)m.range_entries;
  hipLaunchKernelGGL(mask_range_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, cls, m.mg, m.nt, m.nrb, n,
                     range);
  return check_launch("mask preparation launch");
}

static int check_mask_shape(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int64_t msb, int64_t msh,
                            int64_t msq, const char* who) {
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "%s: sizes must be positive", who);
  SAGE_REQUIRE(H % Hkv == 0, "%s: heads %d not a multiple of kv heads %d", who, H, Hkv);
  if (!head_dim_ok(D)) return fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 96, 128, 256)", who, D);
  if (causal && Sq > Skv) return fail(SAGE_ERR_UNSUPPORTED, "%s: causal attention needs q_len <= kv_len", who);
  SAGE_REQUIRE(msb >= 0 && msh >= 0 && msq >= 0, "%s: mask strides (%lld, %lld, %lld) must be non-negative", who,
               (long long)msb, (long long)msh, (long long)msq);
  const MaskShape m = mask_shape(B, H, Sq, Skv, msb, msh, msq, causal);
  // the kernel addresses one (batch, head) slice of the bits with a 32-bit byte offset
  SAGE_REQUIRE((int64_t)m.mq * m.nt * 8 < (1ll << 31), "%s: mask of %d rows x %d keys too large", who, Sq, Skv);
  SAGE_REQUIRE(m.cls_entries < (1ll << 31) && (int64_t)B * H * ((Sq + 127) / 128) * 16 < (1ll << 31),
               "%s: too many query tiles", who);
  SAGE_REQUIRE((int64_t)layout_dim(D) * kv_pad(Skv) < (1ll << 31), "%s: kv_len %d too long", who, Skv);
  return SAGE_OK;
}

}  // namespace sage

extern "C" {

int sage_mask_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int64_t msb, int64_t msh,
                        int64_t msq, int64_t* workspace_bytes) {
  sage::clear_error();
  const char* who = "sage_mask_workspace";
  SAGE_REQUIRE(workspace_bytes != nullptr, "%s: workspace_bytes is NULL", who);
  int rc = sage::check_mask_shape(B, H, Hkv, Sq, Skv, D, causal, msb, msh, msq, who);
  if (rc) return rc;
  const sage::MaskShape m = sage::mask_shape(B, H, Sq, Skv, msb, msh, msq, causal);
  sage::MaskWorkspace w;
  if ((rc = sage::mask_workspace(B, H, Hkv, Sq, Skv, D, m, &w))) return rc;
  *workspace_bytes = w.total;
  return SAGE_OK;
}

int sage_forward_masked(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                        int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out, int64_t osb,
                        int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal,
                        float qs_mul, const void* mask, int64_t msb, int64_t msh, int64_t msq, int8_t* q8, float* qs,
                        int8_t* k8, float* ks, uint8_t* v8t, float* vs, void* workspace, int64_t workspace_bytes,
                        void* stream) {
  sage::clear_error();
  const char* who = "sage_forward_masked";
  // everything is validated before the first launch, so a bad call leaves the stream untouched
  int rc = sage::check_mask_shape(B, H, Hkv, Sq, Skv, D, causal, msb, msh, msq, who);
  if (rc) return rc;
  if (dtype != SAGE_DTYPE_BF16 && dtype != SAGE_DTYPE_F16)
    return sage::fail(SAGE_ERR_UNSUPPORTED, "%s: dtype code %d (bf16=0, f16=1)", who, dtype);
  SAGE_REQUIRE(mask != nullptr, "%s: mask is NULL", who);
  SAGE_REQUIRE(out != nullptr && sage::aligned16(out), "%s: out must be non-NULL and 16-byte aligned", who);
  SAGE_REQUIRE(osb % 8 == 0 && oss % 8 == 0 && osh % 8 == 0 && osb >= 0 && oss >= 0 && osh >= 0,
               "%s: out strides must be non-negative multiples of 8 elements", who);
  SAGE_REQUIRE(workspace != nullptr && ((uintptr_t)workspace & 255u) == 0,
               "%s: workspace must be non-NULL and 256-byte aligned", who);
  const sage::MaskShape m = sage::mask_shape(B, H, Sq, Skv, msb, msh, msq, causal);
  sage::MaskWorkspace w;
  if ((rc = sage::mask_workspace(B, H, Hkv, Sq, Skv, D, m, &w))) return rc;
  SAGE_REQUIRE(workspace_bytes >= w.total, "%s: workspace of %lld bytes, the call needs %lld", who,
               (long long)workspace_bytes, (long long)w.total);
  // q / k / v and the intermediates are checked by the quantization step before it launches anything
  char* ws = static_cast<char*>(workspace);
  uint32_t* bits = reinterpret_cast<uint32_t*>(ws + w.bits);
  int* cls = reinterpret_cast<int*>(ws + w.cls);
  int2* range = reinterpret_cast<int2*>(ws + w.range);
  float* vpart = reinterpret_cast<float*>(ws + w.vpart);
  if ((rc = sage::forward_quant_impl(q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, B, H, Hkv, Sq, Skv, D, dtype,
                                     qs_mul, q8, qs, vpart, k8, ks, v8t, vs, stream)))
    return rc;
  if ((rc = sage::launch_mask_prep(mask, msb, msh, msq, Sq, Skv, causal, m, bits, cls, range, (hipStream_t)stream)))
    return rc;
  const sage::MaskTabs mt{bits,
                          cls,
                          range,
                          m.mb > 1 ? (int64_t)m.mh * m.mq * m.nt * 2 : 0,
                          m.mh > 1 ? (int64_t)m.mq * m.nt * 2 : 0,
                          m.mq > 1 ? (int64_t)m.nt * 2 : 0,
                          m.mb > 1 ? (int64_t)m.mh * m.mg * m.nt : 0,
                          m.mh > 1 ? (int64_t)m.mg * m.nt : 0,
                          m.mg > 1 ? (int64_t)m.nt : 0,
                          m.mb > 1 ? (int64_t)m.mh * m.nrb : 0,
                          m.mh > 1 ? (int64_t)m.nrb : 0,
                          m.mg,
                          m.nrb};
  return sage::attn_mask_impl(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, dtype, &mt,
                              w.attn ? workspace : nullptr, stream);
}

}  // extern "C"
