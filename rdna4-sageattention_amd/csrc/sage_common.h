// Device helpers shared by the gfx950 SageAttention kernels (wave64, CDNA4).
//
// Numerics contract (mirrored bit for bit by oracle/sage_oracle.py):
//  * Hadamard rotation: float64 fast Walsh-Hadamard transform, stage bit 0 first, butterfly (a, b) -> (a + b, a - b),
//    then one float32 rounding.  The stages commute, so lanes may own any contiguous slice as long as the stage
//    order is kept.
//  * x / s with s shared by a whole row or block: r = RN(1 / s) once, then y0 = x * r, e = fma(-y0, s, x),
//    y = fma(e, r, y0), which equals the IEEE quotient RN(x / s) (Markstein's correction with a correctly rounded
//    reciprocal; the remainder e is exact because y0 is within one ulp of x / s).
//  * int8 rounding: trunc(y >= 0 ? fp32(y + 0.5) : fp32(y - 0.5)) (kernel_build/sage_quant.py:44, :65).
//  * fp32 -> E4M3FN: round to nearest even with subnormals, inputs already clamped to +-448.
// Every translation unit is compiled with -ffp-contract=off: the only fused multiply-adds are the explicit ones.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace sage {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

enum { DT_BF16 = 0, DT_F16 = 1 };

// ---- element <-> float -------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float f16_lo(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w & 0xFFFF))); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w >> 16))); }

template <int DT> __device__ __forceinline__ float elem_lo(uint32_t w) { return DT == DT_BF16 ? bf16_lo(w) : f16_lo(w); }
template <int DT> __device__ __forceinline__ float elem_hi(uint32_t w) { return DT == DT_BF16 ? bf16_hi(w) : f16_hi(w); }

// float32 -> bf16 / fp16 bits, round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) { return (uint32_t)__half_as_ushort(__float2half_rn(f)); }
template <int DT> __device__ __forceinline__ uint32_t f32_to_out_bits(float f) {
  return DT == DT_BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
}

// ---- cross-lane moves -------------------------------------------------------------------------------------------
// DPP quad_perm selectors: lane i of each quad reads lane sel[i].
constexpr int DPP_QUAD_XOR1 = 0xB1;  // [1, 0, 3, 2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // [2, 3, 0, 1]
constexpr int DPP_ROW_ROR4 = 0x124;  // each 16-lane row rotated by 4 lanes
constexpr int DPP_ROW_ROR8 = 0x128;  // each 16-lane row rotated by 8 lanes

// (quad_perm reads a valid lane for every lane, so the DPP "old" value is never used: mov_dpp needs no copy of it)
template <int CTRL> __device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}
template <int CTRL> __device__ __forceinline__ double dpp_f64(double x) {
  const int lo = __double2loint(x), hi = __double2hiint(x);
  const int plo = __builtin_amdgcn_mov_dpp(lo, CTRL, 0xF, 0xF, false);
  const int phi = __builtin_amdgcn_mov_dpp(hi, CTRL, 0xF, 0xF, false);
  return __hiloint2double(phi, plo);
}

// Maximum over the wave of a non-negative float, as a wave-uniform value: quad DPP exchanges, two rotations inside
// each 16-lane row, then the four rows' values read into scalar registers (non-negative floats order like their
// bit patterns as unsigned ints)
__device__ __forceinline__ float wave_max_pos(float x) {
  x = fmaxf(x, dpp_f32<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp_f32<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp_f32<DPP_ROW_ROR4>(x));
  x = fmaxf(x, dpp_f32<DPP_ROW_ROR8>(x));
  const uint32_t b = __float_as_uint(x);
  const uint32_t r0 = __builtin_amdgcn_readlane(b, 0), r1 = __builtin_amdgcn_readlane(b, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(b, 32), r3 = __builtin_amdgcn_readlane(b, 48);
  return __uint_as_float(max(max(r0, r1), max(r2, r3)));
}

// A scheduling fence for the 32 values of a wave's tile (float[2][16]): every value passes through this empty
// statement, so the instructions producing them issue before it and those consuming them after it.
#define SAGE_PHASE_FENCE(a)                                                                                \
  asm volatile("" : "+v"(a[0][0]), "+v"(a[0][1]), "+v"(a[0][2]), "+v"(a[0][3]), "+v"(a[0][4]), "+v"(a[0][5]), \
                     "+v"(a[0][6]), "+v"(a[0][7]), "+v"(a[0][8]), "+v"(a[0][9]), "+v"(a[0][10]), "+v"(a[0][11]), \
                     "+v"(a[0][12]), "+v"(a[0][13]), "+v"(a[0][14]), "+v"(a[0][15]), "+v"(a[1][0]), "+v"(a[1][1]), \
                     "+v"(a[1][2]), "+v"(a[1][3]), "+v"(a[1][4]), "+v"(a[1][5]), "+v"(a[1][6]), "+v"(a[1][7]), \
                     "+v"(a[1][8]), "+v"(a[1][9]), "+v"(a[1][10]), "+v"(a[1][11]), "+v"(a[1][12]), "+v"(a[1][13]), \
                     "+v"(a[1][14]), "+v"(a[1][15]))

// Wait until at most N of this wave's vector memory operations are outstanding (they complete in issue order)
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 15, "vmcnt immediate");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier between K / V tiles.  The tile buffers are written only by direct global -> LDS loads, which
// the loops wait for explicitly (vmcnt), and read by ds_reads, which complete before the tile's MFMAs use them; so
// the barrier needs no memory fence.  __syncthreads()'s fence would make the compiler wait for every outstanding
// direct load (vmcnt(0)), including the prefetch of a later tile.  The empty asm statements keep the compiler from
// moving LDS accesses across the barrier.
__device__ __forceinline__ void tile_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Combine a value with the one held by lane (lane ^ 32), in every lane.  v_permlane32_swap_b32 on two copies of x
// leaves r[0] = x[lane mod 32] and r[1] = x[lane mod 32 + 32] in every lane: one VALU op, where a ds_bpermute would
// be an LDS round trip.  max and + are commutative, so both halves get the same bits in the same order as
// op(x[lane], x[lane ^ 32]) would give them.
__device__ __forceinline__ float max_xor32_f32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// One v_permlane32_swap_b32 on two per-lane partial maxima a (block 0) and b (block 1) of rows held by lanes l and
// l ^ 32: the result is row (l mod 32)'s full maximum of a in lanes 0-31 and of b in lanes 32-63.
__device__ __forceinline__ int halves_max_i32(int a, int b) {
  const auto r = __builtin_amdgcn_permlane32_swap((unsigned)a, (unsigned)b, false, false);
  return max((int)r[0], (int)r[1]);
}
__device__ __forceinline__ float halves_max_f32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The inverse exchange: from x (block 0's value in lanes 0-31, block 1's in lanes 32-63, per row l mod 32), both
// values in every lane: lo = block 0's, hi = block 1's.
__device__ __forceinline__ void halves_split_f32(float x, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32_f32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- Hadamard (float64 FWHT) -----------------------------------------------------------------------------------
// x holds EPL consecutive elements of a row whose other slices sit in the 1 / 2 / 4 neighbouring lanes of a quad
// (LANES = D / EPL lanes per row, aligned to quads).  In-lane stages first, then the cross-lane stages, so the
// global stage order is bit 0, 1, 2, ...
template <int EPL, int LANES>
__device__ __forceinline__ void fwht_f64(double (&x)[EPL], int quad_lane) {
#pragma unroll
  for (int s = 1; s < EPL; s <<= 1) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      if (!(i & s)) {
        const double a = x[i], b = x[i + s];
        x[i] = a + b;
        x[i + s] = a - b;
      }
    }
  }
  if (LANES >= 2) {
    // the lane with the stage bit clear holds a and computes a + b; the other holds b and computes a - b
    const double sg = (quad_lane & 1) ? -1.0 : 1.0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) x[i] = __builtin_fma(sg, x[i], dpp_f64<DPP_QUAD_XOR1>(x[i]));
  }
  if (LANES >= 4) {
    const double sg = (quad_lane & 2) ? -1.0 : 1.0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) x[i] = __builtin_fma(sg, x[i], dpp_f64<DPP_QUAD_XOR2>(x[i]));
  }
}

// max over the LANES lanes of a quad-aligned row group
template <int LANES> __device__ __forceinline__ float row_max(float v) {
  if (LANES >= 2) v = fmaxf(v, dpp_f32<DPP_QUAD_XOR1>(v));
  if (LANES >= 4) v = fmaxf(v, dpp_f32<DPP_QUAD_XOR2>(v));
  return v;
}

// ---- quantization helpers ---------------------------------------------------------------------------------------
// RN(x / s) given r = RN(1 / s)
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  const float y0 = x * r;
  const float e = __builtin_fmaf(-y0, s, x);
  return __builtin_fmaf(e, r, y0);
}

// trunc(y >= 0 ? fp32(y + 0.5) : fp32(y - 0.5)); copysign gives -0.5 only for y < 0 or y = -0, and -0 - 0.5 truncates
// to 0 like +0 + 0.5 does, so one bitfield insert replaces the compare and select
__device__ __forceinline__ int round_half_away(float y) {
  const float t = y + __builtin_copysignf(0.5f, y);
  return (int)t;  // v_cvt_i32_f32 truncates toward zero
}

// float32 in [-448, 448] -> E4M3FN byte, round to nearest even, subnormals kept
__device__ __forceinline__ uint32_t f32_to_e4m3(float y) {
  const uint32_t u = __float_as_uint(y);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = fabsf(y);
  uint32_t code;
  if (a >= 0.015625f) {  // 2^-6, smallest normal E4M3
    const uint32_t ab = __float_as_uint(a);
    const uint32_t r = (ab + 0x7FFFFu + ((ab >> 20) & 1u)) >> 20;
    code = r - ((127u - 7u) << 3);
  } else {
    code = (uint32_t)__builtin_rintf(a * 512.0f);  // m * 2^-9, m in 0..8 (8 is the smallest normal code)
  }
  return code | sign;
}

// ---- head dims --------------------------------------------------------------------------------------------------
// Head dims of the path (kernel_build/build_kernels.py:26-41): power-of-two dims are rotated by a Hadamard block of
// RB = min(D, 128) channels (block-diagonal for D = 256, kernel_build/sage_quant.py:18-30); D = 96 is not rotated
// and its int8 / E4M3 rows are stored zero-padded to DP = 128 channels, so the d128 attention kernel runs it.
template <int D> struct HeadDim {
  static constexpr int DP = D == 96 ? 128 : D;                // channels of the Q8 / K8 / V8T / VS layouts
  static constexpr bool ROT = (D & (D - 1)) == 0;             // Hadamard rotation
  static constexpr int RB = D < 128 ? D : 128;                // rotation block
  static constexpr int EPL = DP / 4;                          // elements per lane, 4 lanes per row
  static constexpr int RLANES = ROT ? RB / EPL : 1;           // lanes per rotation block
};

// ---- misc -------------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)(d & 0xFF) << 24);
}

// Map a hardware workgroup id to a logical one so that a contiguous logical range lands on one XCD.  Workgroups are
// dispatched round-robin over the 8 XCDs; XCD x receives ids x, x + 8, x + 16, ...
__device__ __forceinline__ int xcd_remap(int id, int total) {
  constexpr int NX = 8;
  const int q = total / NX, r = total % NX;
  const int x = id % NX, i = id / NX;
  return x * q + (x < r ? x : r) + i;
}

// Causal launches (tiles of different lengths): the (batch, head) pair and query tile of workgroup `id` among
// bh_count * q_tiles.  When the pairs divide over the 8 XCDs, XCD x keeps its own group of pairs (nh of them: their K/V
// stays in its L2) and takes their tiles longest first across the group: the last query tile of every pair, then the
// one before, and so on, so that every pair's short tiles come last.  Otherwise: each XCD a contiguous range, longest
// first within each pair.
__device__ __forceinline__ void causal_tile(int id, int bh_count, int q_tiles, int& bh, int& qt) {
  constexpr int NX = 8;
  if (bh_count % NX == 0) {
    const int nh = bh_count / NX, x = id % NX, i = id / NX;
    bh = x * nh + i % nh;
    qt = q_tiles - 1 - i / nh;
  } else {
    const int logical = xcd_remap(id, bh_count * q_tiles);
    bh = logical / q_tiles;
    qt = q_tiles - 1 - logical % q_tiles;
  }
}

}  // namespace sage
