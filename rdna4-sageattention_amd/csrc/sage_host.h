// Host-side helpers shared by the C-ABI entry points: error reporting and argument checks.
// Nothing here touches the GPU, so argument validation works (and is tested) on machines without one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>

#include "../../include/sage_capi.h"

namespace sage {

// thread-local message behind sage_last_error(); returns `code` for convenient `return fail(...)`
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t err, const char* what);
void clear_error();

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

#define SAGE_REQUIRE(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::sage::fail(SAGE_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define SAGE_HIP_CHECK(expr, what)                               \
  do {                                                           \
    hipError_t _e = (expr);                                      \
    if (_e != hipSuccess) return ::sage::hip_fail(_e, what);     \
  } while (0)

// after a kernel launch: report launch-configuration errors without synchronising
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  return SAGE_OK;
}

// the factor folded into the Q scales (sm_scale * sqrt(head_dim)): the attention assumes positive, finite row
// scales (its row maxima are taken on the raw integer scores), so anything else is rejected (NaN fails both tests)
inline int check_qs_mul(float qs_mul, const char* who) {
  SAGE_REQUIRE(qs_mul > 0.0f && qs_mul <= 3.402823466e38f, "%s: qs_mul must be positive and finite (got %g)", who,
               (double)qs_mul);
  return SAGE_OK;
}

// head dims of the path, and the channel count of their int8 / E4M3 layouts (96 is stored zero-padded to 128)
__host__ __device__ constexpr bool head_dim_ok(int d) { return d == 64 || d == 96 || d == 128 || d == 256; }
__host__ __device__ constexpr int layout_dim(int d) { return d == 96 ? 128 : d; }

// padded KV length used by every K8 / KS / V8T layout
inline int kv_pad(int skv) { return (skv + SAGE_KV_PAD - 1) / SAGE_KV_PAD * SAGE_KV_PAD; }

// Boolean attention mask as the attention kernel reads it (built by mask_prep_block and mask_range_block of
// sage_mask.h, inside the two quantization launches).
// bits: one 32-bit word per (row, 64-key tile, lane half hf): bit 16 kb + v is the visibility of the key that the QK
// accumulator gives lane (query, hf) in register v of 32-key block kb, i.e. key 64 t + 32 kb + 8 (v / 4) + 4 hf + v % 4.
// cls: per (32-row group, tile) 0 = no row sees a key of the tile, 1 = every row sees every key (with a zero bias),
// 2 = mixed visibility, 3 = an additive bias (values in `bias`, -inf where masked).  range:
// per 128-row block, the first tile and one past the last tile of class != 0 in any of its four groups.  Strides are
// in words / entries; 0 broadcasts (a mask without a batch, head or row axis).  The three tables are also passed to
// the kernel as __restrict__ arguments of their own (global loads of the words, scalar loads of classes and ranges).
struct MaskTabs {
  const uint32_t* bits;
  const int* cls;
  const int2* range;
  const uint16_t* bias;   // additive masks: 32 values per bits word (class-3 tiles), strides = the bits' x 32
  int64_t bsb, bsh, bsq;  // bits: batch, head, row strides (a tile adds 2 words)
  int64_t csb, csh, csg;  // cls: batch, head, 32-row group strides (a tile adds 1)
  int64_t rsb, rsh;       // range: batch, head strides (a 128-row block adds 1)
  int groups;             // 32-row groups of cls (1 when the mask has no row axis)
  int rblocks;            // 128-row blocks of range (1 when the mask has no row axis)
};

}  // namespace sage
