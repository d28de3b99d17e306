// C ABI glue: error reporting, queries, the one-call forward (quantizers -> attention) and its allocation-free
// variant on the library's own device scratch array.
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "sage_host.h"

namespace sage {

static thread_local char g_err[512] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  snprintf(g_err, sizeof(g_err), "%s failed: %s (%d)", what, hipGetErrorString(err), (int)err);
  return SAGE_ERR_HIP;
}

void clear_error() { g_err[0] = 0; }

int quant_q_impl(const void*, int64_t, int64_t, int64_t, int, int, int, int, int, float, int8_t*, float*, void*);
int v_amax_impl(const void*, int64_t, int64_t, int64_t, int, int, int, int, int, float*, void*);
int quant_kv_impl(const void*, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, int64_t, int, int, int, int,
                  int, const float*, int8_t*, float*, uint8_t*, void*);
int attn_impl(const int8_t*, const float*, const int8_t*, const float*, const uint8_t*, const float*, void*, int64_t,
              int64_t, int64_t, int, int, int, int, int, int, int, int, float*, void*, int64_t, void*);
int attn_plan_impl(int, int, int, int, int, int, int*, int*, int64_t*);
int attn_args_check(const int8_t*, const float*, const int8_t*, const float*, const uint8_t*, const float*, const void*,
                    int64_t, int64_t, int64_t, int, int, int, int, int, int, int, int, const char*);
int64_t vamax_partial_bytes(int B, int Hkv, int Skv, int D);
int forward_inputs_check(const void*, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, int64_t, const void*,
                         int64_t, int64_t, int64_t, int, int, int, int, int, int, int, const char*);
struct MaskPrep;
int forward_quant_impl(const void*, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, int64_t, const void*,
                       int64_t, int64_t, int64_t, int, int, int, int, int, int, int, float, int8_t*, float*, float*,
                       int8_t*, float*, uint8_t*, float*, const MaskPrep*, void*);

// sage_forward's workspace: the attention plan's partial state, then (256-byte aligned) the per-chunk V maxima.
static int forward_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int64_t* attn_bytes,
                             int64_t* total) {
  int rc = attn_plan_impl(B, H, Sq, Skv, D, causal, nullptr, nullptr, attn_bytes);
  if (rc) return rc;
  *total = (*attn_bytes + 255) / 256 * 256 + vamax_partial_bytes(B, Hkv, Skv, D);
  return SAGE_OK;
}

// ---- scratch of sage_forward_noalloc ----------------------------------------------------------------------------
// Device memory for the intermediates and workspace of sage_forward_noalloc, for callers that cannot allocate.  Each
// GPU the library runs on holds its own copy until the process ends.  In host code `scratch` is only a stand-in for
// the symbol: its device address, different on every GPU, comes from hipGetSymbolAddress (scratch_base) and only that
// address is ever handed to kernels.
static __device__ __align__(256) uint8_t scratch[SAGE_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static void* g_scratch[MAX_DEVICES] = {};
static std::mutex g_scratch_mu;

// The current device's address of `scratch`, looked up once per device with that device current.
static int scratch_base(void** base) {
  int dev = 0;
  SAGE_HIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
  SAGE_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "sage_forward_noalloc: device %d beyond the %d the library tracks", dev,
               MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    SAGE_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    SAGE_REQUIRE(ptr != nullptr && ((uintptr_t)ptr & 255u) == 0, "sage_forward_noalloc: scratch address %p", ptr);
    g_scratch[dev] = ptr;
  }
  *base = g_scratch[dev];
  return SAGE_OK;
}

static int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

}  // namespace sage

extern "C" {

int sage_abi_version(void) { return 6; }

const char* sage_last_error(void) { return sage::g_err; }

int sage_kv_pad(int skv) { return skv <= 0 ? 0 : sage::kv_pad(skv); }

int sage_layout_dim(int head_dim) { return sage::head_dim_ok(head_dim) ? sage::layout_dim(head_dim) : 0; }

const char* sage_manifest_json(void) {
  return "{\"arch\": \"gfx950\", \"head_dims\": [64, 96, 128, 256], \"layout_dims\": [64, 128, 128, 256], "
         "\"rotation_block\": [64, 0, 128, 128], \"dtypes\": [\"bf16\", \"f16\"], "
         "\"kv_block\": 32, \"kv_pad\": 128, "
         "\"quant_q\": {\"rows_per_block\": 64, \"threads\": 256, \"lanes_per_row\": 4, \"rotation\": \"fwht_f64\"}, "
         "\"quant_kv\": {\"rows_per_block\": 128, \"threads\": 256}, "
         "\"v_amax\": {\"rows_per_block\": 256, \"threads\": 256}, "
         "\"attn\": {\"block_m\": 128, \"block_n\": 64, \"threads\": 256, \"waves_per_simd\": {\"d64\": 3, \"d128\": 3, \"d256\": 2}, "
         "\"max_kv_chunks\": 16, "
         "\"mfma_qk\": \"v_mfma_i32_32x32x32_i8\", \"mfma_pv\": \"v_mfma_f32_32x32x64_f8f6f4\", "
         "\"variants\": [\"d64\", \"d96 (128-channel layout, 96 channels of MFMA work)\", \"d128\", \"d256\"], \"causal\": true, \"gqa\": true, \"out_dtypes\": [\"bf16\", \"f16\"]}, "
         "\"varlen\": {\"meta_threads\": 1024, \"sort_bins\": 2048, \"kv_rows_per_sequence\": \"multiple of 128\"}, "
         "\"mask\": {\"dtypes\": [\"bool\", \"bf16 (additive)\", \"f16 (additive)\"], \"broadcast\": [\"batch\", \"head\", \"row\"], \"causal\": \"folded into the bits\", "
         "\"tables\": [\"bits u32 per (row, 64-key tile, lane half)\", \"class per (32 rows, tile)\", \"tile range per 128 rows\", \"bias values of class-3 tiles (float masks)\"], "
         "\"fully_masked_row\": 0}, "
         "\"lse\": {\"head_dims\": [64, 128], \"block_m\": 128, \"block_n\": 64, \"threads\": 256, \"mfma\": \"v_mfma_f32_32x32x16_{bf16,f16}\", "
         "\"causal\": \"bottom-right, q_len <= kv_len\"}}";
}

int sage_forward_workspace(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, int64_t* workspace_bytes) {
  sage::clear_error();
  SAGE_REQUIRE(workspace_bytes != nullptr, "sage_forward_workspace: workspace_bytes is NULL");
  SAGE_REQUIRE(Hkv > 0 && H % Hkv == 0, "sage_forward_workspace: heads %d not a multiple of kv heads %d", H, Hkv);
  int64_t attn = 0;
  return sage::forward_workspace(B, H, Hkv, Sq, Skv, D, causal, &attn, workspace_bytes);
}

int sage_forward(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                 int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out, int64_t osb, int64_t oss,
                 int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal, float qs_mul,
                 int8_t* q8, float* qs, int8_t* k8, float* ks, uint8_t* v8t, float* vs, void* workspace,
                 int64_t workspace_bytes, void* stream) {
  sage::clear_error();
  // validate everything before the first launch so a bad call leaves the stream untouched
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "sage_forward: sizes must be positive");
  SAGE_REQUIRE(H % Hkv == 0, "sage_forward: heads %d not a multiple of kv heads %d", H, Hkv);
  if (!sage::head_dim_ok(D))
    return sage::fail(SAGE_ERR_UNSUPPORTED, "sage_forward: head_dim %d (supported 64, 96, 128, 256)", D);
  if (causal && Sq > Skv) return sage::fail(SAGE_ERR_UNSUPPORTED, "sage_forward: causal attention needs q_len <= kv_len");
  int rc = sage::forward_inputs_check(q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, B, H, Hkv, Sq, Skv, D, dtype,
                                      "sage_forward");
  if (rc) return rc;
  if ((rc = sage::check_qs_mul(qs_mul, "sage_forward"))) return rc;
  // the attention step's checks (its size limits, the output, the intermediates) before the quantizers launch
  if ((rc = sage::attn_args_check(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, causal, dtype,
                                  "sage_forward")))
    return rc;
  if (workspace == nullptr) {
    // no workspace: V maxima by atomics (four quantization launches) and every attention tile whole
    if ((rc = sage::v_amax_impl(v, vsb, vss, vsh, B, Hkv, Skv, D, dtype, vs, stream))) return rc;
    if ((rc = sage::quant_q_impl(q, qsb, qss, qsh, B, H, Sq, D, dtype, qs_mul, q8, qs, stream))) return rc;
    if ((rc = sage::quant_kv_impl(k, ksb, kss, ksh, v, vsb, vss, vsh, B, Hkv, Skv, D, dtype, vs, k8, ks, v8t, stream)))
      return rc;
    return sage::attn_impl(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, causal, dtype, nullptr,
                           nullptr, 0, stream);
  }
  int64_t attn_bytes = 0, need = 0;
  if ((rc = sage::forward_workspace(B, H, Hkv, Sq, Skv, D, causal, &attn_bytes, &need))) return rc;
  SAGE_REQUIRE(workspace_bytes >= need, "sage_forward: workspace of %lld bytes, the plan needs %lld",
               (long long)workspace_bytes, (long long)need);
  SAGE_REQUIRE(((uintptr_t)workspace & 255u) == 0, "sage_forward: workspace must be 256-byte aligned");
  float* vpart = reinterpret_cast<float*>(static_cast<char*>(workspace) + (attn_bytes + 255) / 256 * 256);
  if ((rc = sage::forward_quant_impl(q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, B, H, Hkv, Sq, Skv, D, dtype,
                                     qs_mul, q8, qs, vpart, k8, ks, v8t, vs, nullptr, stream)))
    return rc;
  return sage::attn_impl(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, causal, dtype, nullptr,
                         attn_bytes ? workspace : nullptr, attn_bytes, stream);
}

int sage_forward_noalloc(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb,
                         int64_t kss, int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, void* out,
                         int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype,
                         int causal, float qs_mul, void* stream) {
  sage::clear_error();
  const char* who = "sage_forward_noalloc";
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "%s: sizes must be positive", who);
  SAGE_REQUIRE(H % Hkv == 0, "%s: heads %d not a multiple of kv heads %d", who, H, Hkv);
  if (!sage::head_dim_ok(D)) return sage::fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 96, 128, 256)", who, D);
  if (causal && Sq > Skv) return sage::fail(SAGE_ERR_UNSUPPORTED, "%s: causal attention needs q_len <= kv_len", who);
  int rc = sage::check_qs_mul(qs_mul, who);
  if (rc) return rc;
  // the intermediates of sage_forward, then its workspace, each 256-byte aligned
  const int64_t dl = sage::layout_dim(D), skp = sage::kv_pad(Skv);
  const int64_t nq = (int64_t)B * H * Sq, nkv = (int64_t)B * Hkv;
  int64_t attn_bytes = 0, ws_bytes = 0;
  if ((rc = sage::forward_workspace(B, H, Hkv, Sq, Skv, D, causal, &attn_bytes, &ws_bytes))) return rc;
  const int64_t o_q8 = 0;
  const int64_t o_qs = o_q8 + sage::align256(nq * dl);
  const int64_t o_k8 = o_qs + sage::align256(nq * 4);
  const int64_t o_ks = o_k8 + sage::align256(nkv * skp * dl);
  const int64_t o_v8t = o_ks + sage::align256(nkv * (skp / SAGE_KV_BLOCK) * 4);
  const int64_t o_vs = o_v8t + sage::align256(nkv * dl * skp);
  const int64_t o_ws = o_vs + sage::align256(nkv * dl * 4);
  const int64_t need = o_ws + ws_bytes;
  if (need > (int64_t)SAGE_NOALLOC_SCRATCH_BYTES)
    return sage::fail(SAGE_ERR_INVALID, "%s: this shape needs %lld bytes of scratch, the library holds %lld "
                      "(use sage_forward with caller-owned buffers)", who, (long long)need,
                      (long long)SAGE_NOALLOC_SCRATCH_BYTES);
  void* base = nullptr;
  if ((rc = sage::scratch_base(&base))) return rc;
  uint8_t* p = static_cast<uint8_t*>(base);
  return sage_forward(q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D,
                      dtype, causal, qs_mul, reinterpret_cast<int8_t*>(p + o_q8), reinterpret_cast<float*>(p + o_qs),
                      reinterpret_cast<int8_t*>(p + o_k8), reinterpret_cast<float*>(p + o_ks), p + o_v8t,
                      reinterpret_cast<float*>(p + o_vs), p + o_ws, ws_bytes, stream);
}

}  // extern "C"
