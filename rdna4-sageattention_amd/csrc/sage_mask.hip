// Attention masks with torch SDPA's semantics (bool: True = attend; float: added to the scaled scores, -inf =
// masked): the tables that the mask variant of attn_kernel reads, and the one-call masked forward.
//
// The reference has no masked kernel: src/rdna4_sage/__init__.py:78-79 sends every call with an attn_mask to torch
// SDPA.  Here the mask is turned, on the GPU and in the call's stream, into
//   bits  one 32-bit word per (mask row, 64-key tile, lane half hf) in the order of the attention kernel's QK
//         accumulator (bit 16 kb + v <-> key 64 t + 32 kb + 8 (v / 4) + 4 hf + v % 4), so the kernel masks a score
//         with one bit extract and one bit select;
//   cls   one entry per (32-row group, tile): 0 = no row sees a key of the tile (the wave skips it), 1 = every row
//         sees every key with a zero bias (the mask-free tile body), 2 = mixed visibility (the bit-masked body),
//         3 = an additive bias (float masks only: the biased body);
//   bias  float masks: the 16-bit values of class-3 tiles in the bits' lane order, 32 per word;
//   range one (first, last + 1) tile pair per 128-row block (an attention workgroup's rows): the tiles outside it
//         are not visited at all.
// Keys past kv_len and, with the causal flag, keys past the bottom-right diagonal are folded into the bits.  The
// tables are built by extra workgroups of the two quantization launches (sage_mask.h), so a masked call has the
// launches of an unmasked one.
#include "sage_mask.h"

namespace sage {

int forward_quant_impl(const void*, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, int64_t, const void*,
                       int64_t, int64_t, int64_t, int, int, int, int, int, int, int, float, int8_t*, float*, float*,
                       int8_t*, float*, uint8_t*, float*, const MaskPrep*, void*);
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
  bool additive;  // a 16-bit float mask: the bias table is needed
};

static MaskShape mask_shape(int B, int H, int Sq, int Skv, int64_t msb, int64_t msh, int64_t msq, int causal,
                            int mask_dtype) {
  MaskShape m;
  m.additive = mask_dtype != SAGE_DTYPE_BOOL;
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
// the ranges, and for a float mask the bias values (each 256-byte aligned).
struct MaskWorkspace {
  int64_t attn, vpart, bits, cls, range, bias, total;
};

static int mask_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, const MaskShape& m, MaskWorkspace* w) {
  int rc = attn_mask_plan_impl(B, H, Sq, Skv, D, &w->attn);
  if (rc) return rc;
  w->vpart = align256(w->attn);
  w->bits = w->vpart + align256(vamax_partial_bytes(B, Hkv, Skv, D));
  w->cls = w->bits + align256(m.bits_words * 4);
  w->range = w->cls + align256(m.cls_entries * 4);
  w->bias = w->range + align256(m.range_entries * 8);
  w->total = w->bias + (m.additive ? align256(m.bits_words * 32 * 2) : 0);
  return SAGE_OK;
}

static int check_mask_shape(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int mask_dtype, int64_t msb,
                            int64_t msh, int64_t msq, const char* who) {
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "%s: sizes must be positive", who);
  SAGE_REQUIRE(H % Hkv == 0, "%s: heads %d not a multiple of kv heads %d", who, H, Hkv);
  if (!head_dim_ok(D)) return fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 96, 128, 256)", who, D);
  if (causal && Sq > Skv) return fail(SAGE_ERR_UNSUPPORTED, "%s: causal attention needs q_len <= kv_len", who);
  SAGE_REQUIRE(msb >= 0 && msh >= 0 && msq >= 0, "%s: mask strides (%lld, %lld, %lld) must be non-negative", who,
               (long long)msb, (long long)msh, (long long)msq);
  if (mask_dtype != SAGE_DTYPE_BOOL && mask_dtype != SAGE_DTYPE_BF16 && mask_dtype != SAGE_DTYPE_F16)
    return fail(SAGE_ERR_UNSUPPORTED, "%s: mask dtype code %d (bool=2, bf16=0, f16=1)", who, mask_dtype);
  const MaskShape m = mask_shape(B, H, Sq, Skv, msb, msh, msq, causal, mask_dtype);
  // the kernel addresses one (batch, head) slice of the bits (and of the bias values: 16x) with a 32-bit byte offset
  SAGE_REQUIRE((int64_t)m.mq * m.nt * (m.additive ? 128 : 8) < (1ll << 31), "%s: mask of %d rows x %d keys too large",
               who, Sq, Skv);
  SAGE_REQUIRE(m.cls_entries < (1ll << 31) && (int64_t)B * H * ((Sq + 127) / 128) * 16 < (1ll << 31),
               "%s: too many query tiles", who);
  SAGE_REQUIRE((int64_t)layout_dim(D) * kv_pad(Skv) < (1ll << 31), "%s: kv_len %d too long", who, Skv);
  return SAGE_OK;
}

}  // namespace sage

extern "C" {

int sage_mask_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int mask_dtype, int64_t msb,
                        int64_t msh, int64_t msq, int64_t* workspace_bytes) {
  sage::clear_error();
  const char* who = "sage_mask_workspace";
  SAGE_REQUIRE(workspace_bytes != nullptr, "%s: workspace_bytes is NULL", who);
  int rc = sage::check_mask_shape(B, H, Hkv, Sq, Skv, D, causal, mask_dtype, msb, msh, msq, who);
  if (rc) return rc;
  const sage::MaskShape m = sage::mask_shape(B, H, Sq, Skv, msb, msh, msq, causal, mask_dtype);
  sage::MaskWorkspace w;
  if ((rc = sage::mask_workspace(B, H, Hkv, Sq, Skv, D, m, &w))) return rc;
  *workspace_bytes = w.total;
  return SAGE_OK;
}

int sage_forward_masked(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                        int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out, int64_t osb,
                        int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal,
                        float qs_mul, const void* mask, int mask_dtype, int64_t msb, int64_t msh, int64_t msq,
                        int8_t* q8, float* qs, int8_t* k8, float* ks, uint8_t* v8t, float* vs, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  sage::clear_error();
  const char* who = "sage_forward_masked";
  // everything is validated before the first launch, so a bad call leaves the stream untouched
  int rc = sage::check_mask_shape(B, H, Hkv, Sq, Skv, D, causal, mask_dtype, msb, msh, msq, who);
  if (rc) return rc;
  if (dtype != SAGE_DTYPE_BF16 && dtype != SAGE_DTYPE_F16)
    return sage::fail(SAGE_ERR_UNSUPPORTED, "%s: dtype code %d (bf16=0, f16=1)", who, dtype);
  if (mask_dtype != SAGE_DTYPE_BOOL && mask_dtype != dtype)
    return sage::fail(SAGE_ERR_UNSUPPORTED, "%s: a float mask must have the inputs' dtype", who);
  SAGE_REQUIRE(mask != nullptr, "%s: mask is NULL", who);
  if ((rc = sage::check_qs_mul(qs_mul, who))) return rc;
  SAGE_REQUIRE(out != nullptr && sage::aligned16(out), "%s: out must be non-NULL and 16-byte aligned", who);
  SAGE_REQUIRE(osb % 8 == 0 && oss % 8 == 0 && osh % 8 == 0 && osb >= 0 && oss >= 0 && osh >= 0,
               "%s: out strides must be non-negative multiples of 8 elements", who);
  SAGE_REQUIRE(workspace != nullptr && ((uintptr_t)workspace & 255u) == 0,
               "%s: workspace must be non-NULL and 256-byte aligned", who);
  const sage::MaskShape m = sage::mask_shape(B, H, Sq, Skv, msb, msh, msq, causal, mask_dtype);
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
  sage::MaskPrep mp;
  mp.mask = mask;
  mp.mdt = mask_dtype;
  mp.msb = msb;
  mp.msh = msh;
  mp.msq = msq;
  mp.mh = m.mh;
  mp.mq = m.mq;
  mp.mg = m.mg;
  mp.nt = m.nt;
  mp.nrb = m.nrb;
  mp.Sq = Sq;
  mp.Skv = Skv;
  mp.causal = causal;
  // a run of 4 keys as one load: 4 bytes (bool) or 8 bytes (16-bit) aligned rows
  const unsigned run_bytes = mask_dtype == SAGE_DTYPE_BOOL ? 4u : 8u;
  mp.a4 = ((uintptr_t)mask % run_bytes) == 0 && msb % 4 == 0 && msh % 4 == 0 && msq % 4 == 0;
  mp.bits = bits;
  mp.bias = m.additive ? reinterpret_cast<uint16_t*>(ws + w.bias) : nullptr;
  mp.cls = cls;
  mp.range = range;
  mp.nrange = (int)m.range_entries;
  mp.prep_blocks = (int)((int64_t)m.mb * m.mh * m.mg * ((m.nt + 3) / 4));
  mp.range_blocks = (mp.nrange + 3) / 4;
  if ((rc = sage::forward_quant_impl(q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, B, H, Hkv, Sq, Skv, D, dtype,
                                     qs_mul, q8, qs, vpart, k8, ks, v8t, vs, &mp, stream)))
    return rc;
  const sage::MaskTabs mt{bits,
                          cls,
                          range,
                          mp.bias,
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
