// Quantization kernels of the gfx950 SageAttention path (HBM-bound streaming kernels).
//
//  quant_q_kernel   Q rows -> Hadamard (float64 FWHT) -> int8, one scale per token   (sage_quant.py:33-48)
//  fill_kernel      clears the V amax buffer (a kernel, not hipMemsetAsync, so the sequence can be graph-captured)
//  v_amax_kernel    per-channel max |v| over a chunk of rows, combined with atomicMax on the fp32 bit pattern
//                   (values are >= 0, so unsigned order == float order)               (_attention.py:120-121)
//  quant_kv_kernel  K rows -> Hadamard -> int8, one scale per 32 keys; V -> E4M3 with the per-channel scale,
//                   transposed through LDS into V8T                                  (sage_quant.py:51-70)
//  quant_qk_vamax_kernel, quant_v_kernel   the same work in sage_forward's two launches
//  quant_varlen_kernel, quant_v_varlen_kernel   packed variable-length batches
//
// Row mapping of the Hadamard kernels: 4 lanes (one quad) per row, each lane owns DP / 4 consecutive elements
// (32 to 128 bytes of bf16 / fp16), so a wave64 rotates 16 rows at a time.  Head dims 64 / 128 rotate over the whole
// row, 256 over two 128-channel blocks (2 lanes each), 96 is not rotated and lane 3 holds the zero padding of its
// 128-channel layout.
#include "sage_common.h"
#include "sage_host.h"
#include "sage_mask.h"

namespace sage {

constexpr int QUAD = 4;

// 16 bytes from p, or zeros when !valid.  p must be dereferenceable either way (callers point invalid lanes at a
// valid row).  The load is unconditional and the zeroing a bitwise AND: with a select the compiler sinks the load
// into a branch, and a run of such loads then becomes one branch and one wait per load instead of all in flight.
__device__ __forceinline__ uint4 load16_or_zero(const void* p, bool valid) {
  uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t m = 0u - (uint32_t)valid;
  w.x &= m;
  w.y &= m;
  w.z &= m;
  w.w &= m;
  return w;
}

// Load EPL consecutive 16-bit elements (EPL * 2 bytes, 16-byte aligned; src dereferenceable even when !valid) and
// widen them to float64 (zeros when !valid).
template <int EPL, int DT>
__device__ __forceinline__ void load_row_slice(const uint16_t* __restrict__ src, bool valid, double (&x)[EPL]) {
#pragma unroll
  for (int k = 0; k < EPL / 8; ++k) {
    const uint4 w = load16_or_zero(src + 8 * k, valid);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[8 * k + 2 * i] = (double)elem_lo<DT>(ws[i]);
      x[8 * k + 2 * i + 1] = (double)elem_hi<DT>(ws[i]);
    }
  }
}

// Quantize EPL rotated values with the shared scale s (reciprocal r) and store them as EPL int8 bytes.
template <int EPL>
__device__ __forceinline__ void quantize_store_i8(const float (&x)[EPL], float s, float r, int8_t* __restrict__ dst,
                                                  bool valid) {
  uint32_t words[EPL / 4];
#pragma unroll
  for (int i = 0; i < EPL / 4; ++i) {
    const int a = round_half_away(div_by_scale(x[4 * i + 0], s, r));
    const int b = round_half_away(div_by_scale(x[4 * i + 1], s, r));
    const int c = round_half_away(div_by_scale(x[4 * i + 2], s, r));
    const int d = round_half_away(div_by_scale(x[4 * i + 3], s, r));
    words[i] = pack4_i8(a, b, c, d);
  }
  if (valid) {
#pragma unroll
    for (int i = 0; i < EPL / 16; ++i)
      reinterpret_cast<uint4*>(dst)[i] = make_uint4(words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]);
  }
}

// ------------------------------------------------------------------------------------------------------------------
// quant_q: grid = (ceil(S / 64) * B * H), block = 256 (4 waves x 16 rows)
// ------------------------------------------------------------------------------------------------------------------
template <int D, int DT>
__device__ __forceinline__ void quant_q_rows(const uint16_t* __restrict__ x, int64_t sb, int64_t ss, int64_t sh, int H,
                                             int S, int row_tiles, float qs_mul, int8_t* __restrict__ q8,
                                             float* __restrict__ qs, int block) {
  using HD = HeadDim<D>;
  constexpr int EPL = HD::EPL;
  const int tile = block % row_tiles;
  const int bh = block / row_tiles;
  const int b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 3;
  const int row = tile * 64 + wave * 16 + (lane >> 2);
  const bool valid = row < S;
  const bool has_ch = j * EPL < D;  // D = 96: lane 3 holds the zero padding of the 128-channel layout
  const uint16_t* src = x + b * sb + (int64_t)(valid ? row : 0) * ss + h * sh + (has_ch ? j * EPL : 0);

  double xd[EPL];
  load_row_slice<EPL, DT>(src, valid && has_ch, xd);
  if (HD::ROT) fwht_f64<EPL, HD::RLANES>(xd, j);
  float xf[EPL];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    xf[i] = (float)xd[i];
    amax = fmaxf(amax, fabsf(xf[i]));
  }
  amax = fmaxf(row_max<QUAD>(amax), 1e-12f);
  const float s = amax / 127.0f;
  const float r = 1.0f / s;
  int8_t* dst = q8 + ((int64_t)bh * S + row) * HD::DP + j * EPL;
  quantize_store_i8<EPL>(xf, s, r, dst, valid);
  // the unnormalised rotation multiplies Q K^T by RB (sage_quant.py:46-47); no rotation, no division
  if (valid && j == 0) qs[(int64_t)bh * S + row] = (HD::ROT ? s / (float)HD::RB : s) * qs_mul;
}

template <int D, int DT>
__global__ __launch_bounds__(256) void quant_q_kernel(const uint16_t* __restrict__ x, int64_t sb, int64_t ss,
                                                      int64_t sh, int H, int S, int row_tiles, float qs_mul,
                                                      int8_t* __restrict__ q8, float* __restrict__ qs) {
  quant_q_rows<D, DT>(x, sb, ss, sh, H, S, row_tiles, qs_mul, q8, qs, blockIdx.x);
}

// ------------------------------------------------------------------------------------------------------------------
// fill / v_amax
// ------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fill_kernel(float* __restrict__ p, int64_t n, float value) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = value;
}

// Per-channel max |v| over rows [row_beg, row_end) of one (batch, kv head): `base` points at channel 0 of row 0.
// Returns the maximum of channel threadIdx.x in threads [0, DP) (0 for an empty range and for the padding channels
// of D = 96).
template <int D, int DT>
__device__ __forceinline__ float vamax_core(const uint16_t* __restrict__ base, int64_t ss, int row_beg, int row_end) {
  constexpr int DP = HeadDim<D>::DP;
  constexpr int LPR = DP / 8;     // lanes per row, 8 elements (16 bytes) each
  constexpr int RPI = 256 / LPR;  // rows per iteration
  __shared__ float red[RPI][DP + 1];
  const int c8 = threadIdx.x % LPR, r0 = threadIdx.x / LPR;
  const uint16_t* cb = base + c8 * 8;
  if (c8 * 8 >= D) row_end = row_beg;  // padding channels: nothing to load
  float m[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) m[i] = 0.0f;
  // eight rows per thread in flight: issue the loads of a group, then reduce them
  constexpr int G = 8;
  for (int row0 = row_beg + r0; row0 < row_end; row0 += G * RPI) {
    uint4 w[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int row = row0 + g * RPI;
      w[g] = load16_or_zero(cb + (int64_t)(row < row_end ? row : row0) * ss, row < row_end);  // row0 < row_end
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t ws[4] = {w[g].x, w[g].y, w[g].z, w[g].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        m[2 * i] = fmaxf(m[2 * i], fabsf(elem_lo<DT>(ws[i])));
        m[2 * i + 1] = fmaxf(m[2 * i + 1], fabsf(elem_hi<DT>(ws[i])));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[r0][c8 * 8 + i] = m[i];
  __syncthreads();
  float a = 0.0f;
  if (threadIdx.x < DP) {
#pragma unroll 8
    for (int r = 0; r < RPI; ++r) a = fmaxf(a, red[r][threadIdx.x]);
  }
  return a;
}

// One block reduces `chunk_rows` rows of one (batch, kv head) to per-channel max |v|.  PARTIAL: store the chunk's
// maxima to out[(bh * chunks + chunk) * DP + d]; otherwise combine into out[bh * DP + d] with atomicMax on the fp32 bit
// pattern (values are >= 0, so unsigned order == float order; out must start at zero).
template <int D, int DT, bool PARTIAL>
__device__ __forceinline__ void vamax_rows(const uint16_t* __restrict__ v, int64_t sb, int64_t ss, int64_t sh,
                                           int Hkv, int S, int chunks, int chunk_rows, float* __restrict__ out,
                                           int block) {
  const int chunk = block % chunks;
  const int bh = block / chunks;
  const int b = bh / Hkv, h = bh % Hkv;
  constexpr int DP = HeadDim<D>::DP;
  const float a = vamax_core<D, DT>(v + b * sb + h * sh, ss, chunk * chunk_rows, min(S, (chunk + 1) * chunk_rows));
  if (threadIdx.x < DP) {
    if (PARTIAL)
      out[((int64_t)bh * chunks + chunk) * DP + threadIdx.x] = a;
    else
      atomicMax(reinterpret_cast<unsigned int*>(out + (int64_t)bh * DP + threadIdx.x), __float_as_uint(a));
  }
}

// grid = (chunks * B * Hkv), block = 256
template <int D, int DT>
__global__ __launch_bounds__(256) void v_amax_kernel(const uint16_t* __restrict__ v, int64_t sb, int64_t ss,
                                                     int64_t sh, int Hkv, int S, int chunks, int chunk_rows,
                                                     float* __restrict__ vs) {
  vamax_rows<D, DT, false>(v, sb, ss, sh, Hkv, S, chunks, chunk_rows, vs, blockIdx.x);
}

// sage_forward's per-chunk V maxima: chunks of at least V_AMAX_ROWS keys, at most V_AMAX_CHUNKS per (batch, kv head),
// so every V block of the second launch reduces at most 16 rows of maxima
constexpr int V_AMAX_ROWS = 512;
constexpr int V_AMAX_CHUNKS = 16;
__host__ __device__ inline int vamax_chunks(int skv) { return min((skv + V_AMAX_ROWS - 1) / V_AMAX_ROWS, V_AMAX_CHUNKS); }
__host__ __device__ inline int vamax_chunk_rows(int skv) { return (skv + vamax_chunks(skv) - 1) / vamax_chunks(skv); }

// ------------------------------------------------------------------------------------------------------------------
// K: Hadamard -> int8 with one scale per 32 keys.
//  64 keys per block, wave w rotates keys [16w, 16w + 16) and the two waves of a 32-key group combine their maxima
//  through LDS.
// ------------------------------------------------------------------------------------------------------------------
// 64 keys: local rows [local0, local0 + 64) of one (batch, kv head), `base` = row 0 of its source; rows >= nvalid
// are zero.  Writes the 64 int8 rows at k8_blk and the two 32-key scales at ks_blk.
template <int D, int DT>
__device__ __forceinline__ void quant_k64_core(const uint16_t* __restrict__ base, int64_t kss, int local0, int nvalid,
                                               int8_t* __restrict__ k8_blk, float* __restrict__ ks_blk) {
  using HD = HeadDim<D>;
  constexpr int EPL = HD::EPL;
  __shared__ float wave_max[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 3;
  const int r = wave * 16 + (lane >> 2);
  const int row = local0 + r;
  const bool valid = row < nvalid;
  const bool has_ch = j * EPL < D;
  const uint16_t* src = base + (int64_t)(valid ? row : 0) * kss + (has_ch ? j * EPL : 0);
  double xd[EPL];
  load_row_slice<EPL, DT>(src, valid && has_ch, xd);
  if (HD::ROT) fwht_f64<EPL, HD::RLANES>(xd, j);
  float xf[EPL];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    xf[i] = (float)xd[i];
    amax = fmaxf(amax, fabsf(xf[i]));
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if (lane == 0) wave_max[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wave_max[wave & ~1], wave_max[wave | 1]), 1e-12f);
  const float s = amax / 127.0f;
  const float rs = 1.0f / s;
  quantize_store_i8<EPL>(xf, s, rs, k8_blk + (int64_t)r * HD::DP + j * EPL, true);
  if (lane == 0 && (wave & 1) == 0) ks_blk[wave >> 1] = s;
  __syncthreads();  // wave_max may be reused by the next call in this workgroup
}

template <int D, int DT>
__device__ __forceinline__ void quant_k_rows64(const uint16_t* __restrict__ k, int64_t ksb, int64_t kss, int64_t ksh,
                                               int Hkv, int S, int Skp, int8_t* __restrict__ k8,
                                               float* __restrict__ ks, int block) {
  const int nblk = Skp / 64;
  const int blk = block % nblk;
  const int bh = block / nblk;
  const int b = bh / Hkv, h = bh % Hkv;
  quant_k64_core<D, DT>(k + b * ksb + h * ksh, kss, blk * 64, S, k8 + ((int64_t)bh * Skp + blk * 64) * HeadDim<D>::DP,
                        ks + (int64_t)bh * (Skp / SAGE_KV_BLOCK) + blk * 2);
}

// ------------------------------------------------------------------------------------------------------------------
// V: E4M3 with the per-channel scale 448 / max(VS, 1e-30), 128 keys per block, transposed through LDS into V8T.
// Core: local rows [local0, local0 + 128) of one (batch, kv head), `base` = row 0 of its source, rows >= nvalid are
// zero.  vchunks == 0: `am_src` holds the (batch, kv head)'s per-channel amax [D].  vchunks > 0: `am_src` holds its
// per-chunk maxima [vchunks][D]; they are reduced and, when vs_out is not NULL, the amax is stored there.  The 128
// transposed keys go to v8t_blk + d * chan_stride (d = channel).
// ------------------------------------------------------------------------------------------------------------------
template <int D, int DT>
__device__ __forceinline__ void quant_v128_core(const uint16_t* __restrict__ base, int64_t vss, int local0, int nvalid,
                                                const float* __restrict__ am_src, int vchunks,
                                                float* __restrict__ vs_out, uint8_t* __restrict__ v8t_blk,
                                                int64_t chan_stride) {
  constexpr int DP = HeadDim<D>::DP;
  constexpr int PITCH = DP + 4;  // LDS row pitch of the [128 keys][DP] E4M3 staging tile
  __shared__ uint8_t vtile[128 * PITCH];
  // ---- V: scale, E4M3, stage [key][d] in LDS ----
  constexpr int LPR = DP / 8;     // lanes per row (8 channels each)
  constexpr int RPI = 256 / LPR;  // rows per pass
  const int c8 = threadIdx.x % LPR, r0 = threadIdx.x / LPR;
  if (c8 * 8 >= D) nvalid = 0;  // padding channels of D = 96: zeros
  // The channel maxima are loaded first and the thread's 128 / RPI rows of V right behind them: loads complete in
  // order, so the maxima's reduction waits for its own few loads and runs while the rows are in flight.
  const uint16_t* vbase = base + c8 * 8;
  float am[8];
  uint4 wv[128 / RPI];
  if (vchunks == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) am[i] = am_src[c8 * 8 + i];  // VS may be only 4-byte aligned (sage_quant_kv)
#pragma unroll
    for (int g = 0; g < 128 / RPI; ++g) {
      const int row = local0 + r0 + g * RPI;
      const bool ok = row < nvalid;
      wv[g] = load16_or_zero(ok ? vbase + (int64_t)row * vss : base, ok);  // base: row 0, channel 0 of the sequence
    }
  } else {
    // the per-chunk maxima are reduced once per block: thread (4-channel group cg, slice cs) takes the maximum of
    // chunks cs, cs + NSL, ..., the slices meet in LDS, and one row of threads reduces them (and stores VS when
    // vs_out is set); every thread then reads its 8 channels.
    constexpr int NCG = DP / 4, NSL = 256 / NCG, PER = (V_AMAX_CHUNKS + NSL - 1) / NSL;
    __shared__ __attribute__((aligned(16))) float vpart_lds[NSL][DP];
    const int cg = threadIdx.x % NCG, cs = threadIdx.x / NCG;
    v4f pc[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i)  // chunks past the last one repeat it, which a maximum does not notice
      pc[i] = *reinterpret_cast<const v4f*>(am_src + (int64_t)min(cs + i * NSL, vchunks - 1) * DP + 4 * cg);
#pragma unroll
    for (int g = 0; g < 128 / RPI; ++g) {
      const int row = local0 + r0 + g * RPI;
      const bool ok = row < nvalid;
      wv[g] = load16_or_zero(ok ? vbase + (int64_t)row * vss : base, ok);
    }
    v4f m4 = pc[0];
#pragma unroll
    for (int i = 1; i < PER; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) m4[e] = fmaxf(m4[e], pc[i][e]);
    *reinterpret_cast<v4f*>(&vpart_lds[cs][4 * cg]) = m4;
    __syncthreads();
    if (cs == 0) {
#pragma unroll
      for (int j = 1; j < NSL; ++j) {
        const v4f o4 = *reinterpret_cast<const v4f*>(&vpart_lds[j][4 * cg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) m4[e] = fmaxf(m4[e], o4[e]);
      }
      *reinterpret_cast<v4f*>(&vpart_lds[0][4 * cg]) = m4;
      if (vs_out != nullptr) *reinterpret_cast<v4f*>(vs_out + 4 * cg) = m4;
    }
    __syncthreads();
    const v4f a0 = *reinterpret_cast<const v4f*>(&vpart_lds[0][c8 * 8]);
    const v4f a1 = *reinterpret_cast<const v4f*>(&vpart_lds[0][c8 * 8 + 4]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      am[i] = a0[i];
      am[4 + i] = a1[i];
    }
  }
  float cs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cs[i] = 448.0f / fmaxf(am[i], 1e-30f);
#pragma unroll
  for (int g = 0; g < 128 / RPI; ++g) {
    const int rr = r0 + g * RPI;
    const uint32_t ws[4] = {wv[g].x, wv[g].y, wv[g].z, wv[g].w};
    float y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[2 * i] = fminf(fmaxf(elem_lo<DT>(ws[i]) * cs[2 * i], -448.0f), 448.0f);
      y[2 * i + 1] = fminf(fmaxf(elem_hi<DT>(ws[i]) * cs[2 * i + 1], -448.0f), 448.0f);
    }
    // hardware E4M3 conversion (round to nearest even, subnormals kept; inputs are within +-448)
    int t0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    t0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], t0, true);
    int t1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
    t1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], t1, true);
    *reinterpret_cast<uint2*>(vtile + rr * PITCH + c8 * 8) = make_uint2((uint32_t)t0, (uint32_t)t1);
  }
  __syncthreads();

  // ---- V: transposed store.  Thread -> (4-channel group cg, 16-key set ksel); key set ksel = 4G + u covers output
  // positions [64G + 16u, +16) of this 128-key block, i.e. keys 64G + 8g + 4h + r with h = u / 2, g = 4(u % 2) + i.
  constexpr int NCG = DP / 4;
  for (int item = threadIdx.x; item < NCG * 8; item += 256) {
    const int ksel = item % 8, cg = item / 8;
    const int G = ksel >> 2, u = ksel & 3, hh = u >> 1;
    uint32_t wd[4][4];  // [chunk i][key r] -> 4 channel bytes
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * (u & 1) + i;
#pragma unroll
      for (int rk = 0; rk < 4; ++rk) {
        const int key = 64 * G + 8 * g + 4 * hh + rk;
        wd[i][rk] = *reinterpret_cast<const uint32_t*>(vtile + key * PITCH + cg * 4);
      }
    }
#pragma unroll
    for (int ci = 0; ci < 4; ++ci) {
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = ((wd[i][0] >> (8 * ci)) & 0xFFu) | (((wd[i][1] >> (8 * ci)) & 0xFFu) << 8) |
               (((wd[i][2] >> (8 * ci)) & 0xFFu) << 16) | (((wd[i][3] >> (8 * ci)) & 0xFFu) << 24);
      }
      const int d = cg * 4 + ci;
      uint8_t* dst = v8t_blk + (int64_t)d * chan_stride + 64 * G + 16 * u;
      *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// dense layout: grid = (Skp / 128) * B * Hkv blocks; vs_out (vchunks > 0) is written by block 0 of each (b, kv head)
template <int D, int DT>
__device__ __forceinline__ void quant_v_rows(const uint16_t* __restrict__ v, int64_t vsb, int64_t vss, int64_t vsh,
                                             int Hkv, int S, int Skp, const float* __restrict__ vs, int vchunks,
                                             float* __restrict__ vs_out, uint8_t* __restrict__ v8t, int block) {
  const int nblk = Skp / 128;
  const int blk = block % nblk;
  const int bh = block / nblk;
  const int b = bh / Hkv, h = bh % Hkv;
  constexpr int DP = HeadDim<D>::DP;
  const float* am_src = vs + (int64_t)bh * (vchunks == 0 ? 1 : vchunks) * DP;
  float* out_row = (vchunks > 0 && blk == 0) ? vs_out + (int64_t)bh * DP : nullptr;
  quant_v128_core<D, DT>(v + b * vsb + h * vsh, vss, blk * 128, S, am_src, vchunks, out_row,
                         v8t + (int64_t)bh * DP * Skp + blk * 128, Skp);
}

// sage_forward's first launch: blocks [0, nv) write per-chunk V maxima (vamax_chunk_rows keys each) to `vpart`,
// blocks [nv, nv + nk) quantize 64 keys of K each, the next nq quantize Q, and sage_forward_masked's mask blocks
// (mp.prep_blocks of them) follow.  The V blocks come first so their longer row loops start early.
// waves per SIMD the first launch asks for: 5 fit the d128 paths in 96 VGPRs (more loads in flight per CU); d256
// holds twice the row slice and stays at the register count it needs
template <int D> constexpr int quant_qk_waves() { return D == 256 ? 1 : 5; }

template <int D, int DT>
__global__ __launch_bounds__(256, quant_qk_waves<D>()) void quant_qk_vamax_kernel(const uint16_t* __restrict__ x, int64_t sb, int64_t ss,
                                                             int64_t sh, int H, int Sq, int row_tiles, float qs_mul,
                                                             int8_t* __restrict__ q8, float* __restrict__ qs,
                                                             const uint16_t* __restrict__ k, int64_t ksb, int64_t kss,
                                                             int64_t ksh, int Skp, int nk, int8_t* __restrict__ k8,
                                                             float* __restrict__ ks, const uint16_t* __restrict__ v,
                                                             int64_t vsb, int64_t vss, int64_t vsh, int Hkv, int Skv,
                                                             int vchunks, int nv, float* __restrict__ vpart, int nq,
                                                             MaskPrep mp) {
  const int blk = blockIdx.x;
  if (blk < nv)
    vamax_rows<D, DT, true>(v, vsb, vss, vsh, Hkv, Skv, vchunks, vamax_chunk_rows(Skv), vpart, blk);
  else if (blk < nv + nk)
    quant_k_rows64<D, DT>(k, ksb, kss, ksh, Hkv, Skv, Skp, k8, ks, blk - nv);
  else if (blk < nv + nk + nq)
    quant_q_rows<D, DT>(x, sb, ss, sh, H, Sq, row_tiles, qs_mul, q8, qs, blk - nv - nk);
  else
    mask_prep_block(mp, blk - nv - nk - nq);
}

// quant_kv (stage entry point): grid = (Skp / 128 * B * Hkv), block = 256; K then V of 128 keys
template <int D, int DT>
__global__ __launch_bounds__(256) void quant_kv_kernel(const uint16_t* __restrict__ k, int64_t ksb, int64_t kss,
                                                       int64_t ksh, const uint16_t* __restrict__ v, int64_t vsb,
                                                       int64_t vss, int64_t vsh, int Hkv, int S, int Skp,
                                                       const float* __restrict__ vs, int8_t* __restrict__ k8,
                                                       float* __restrict__ ks, uint8_t* __restrict__ v8t) {
  quant_k_rows64<D, DT>(k, ksb, kss, ksh, Hkv, S, Skp, k8, ks, 2 * blockIdx.x);
  quant_k_rows64<D, DT>(k, ksb, kss, ksh, Hkv, S, Skp, k8, ks, 2 * blockIdx.x + 1);
  quant_v_rows<D, DT>(v, vsb, vss, vsh, Hkv, S, Skp, vs, 0, nullptr, v8t, blockIdx.x);
}

// sage_forward's second launch: V (blocks [0, nvb)), reducing the per-chunk maxima of the first; then the mask
// range blocks of sage_forward_masked (mp.range_blocks), which read the classes the first launch wrote
template <int D, int DT>
__global__ __launch_bounds__(256) void quant_v_kernel(const uint16_t* __restrict__ v, int64_t vsb, int64_t vss,
                                                      int64_t vsh, int Hkv, int S, int Skp,
                                                      const float* __restrict__ vpart, int vchunks,
                                                      float* __restrict__ vs, uint8_t* __restrict__ v8t, int nvb,
                                                      MaskPrep mp) {
  if ((int)blockIdx.x < nvb)
    quant_v_rows<D, DT>(v, vsb, vss, vsh, Hkv, S, Skp, vpart, vchunks, vs, v8t, blockIdx.x);
  else
    mask_range_block(mp, blockIdx.x - nvb);
}

// ------------------------------------------------------------------------------------------------------------------
// Packed variable-length sequences.  Q is quantized as one sequence of TQ tokens ([H][TQ] rows: the per-token scale
// does not depend on the sequence).  K8 / KS / V8T use a padded packed layout: sequence b's keys occupy rows
// [kp[b], kp[b] + pad128(len_b)) of each kv head's TKP rows, so every 32-key scale block and every 64-key attention
// tile lies inside one sequence, as in a separate call per sequence.  ktab[g] is the sequence that owns padded
// 128-key block g (-1 past the last one).  vs [batch][Hkv][D] must be zero before the first launch.
// ------------------------------------------------------------------------------------------------------------------
struct VarlenKeys {
  const int* cu_k;  // [batch + 1] token offsets of the sequences in k / v
  const int* kp;    // [batch + 1] padded row offsets
  const int* ktab;  // [TKP / 128] owner of each padded 128-key block
};

// first launch: blocks [0, nv) per-channel V maxima of one padded 128-key block (atomicMax into vs), [nv, nv + nk)
// K of one padded 64-key block, the rest Q.  nv = Hkv * TKP / 128, nk = Hkv * TKP / 64.
template <int D, int DT>
__global__ __launch_bounds__(256) void quant_varlen_kernel(const uint16_t* __restrict__ x, int64_t qss, int64_t qsh,
                                                           int H, int TQ, int row_tiles, float qs_mul,
                                                           int8_t* __restrict__ q8, float* __restrict__ qs,
                                                           const uint16_t* __restrict__ k, int64_t kss, int64_t ksh,
                                                           const uint16_t* __restrict__ v, int64_t vss, int64_t vsh,
                                                           int Hkv, int TKP, VarlenKeys vk, int8_t* __restrict__ k8,
                                                           float* __restrict__ ks, float* __restrict__ vs) {
  const int nv = Hkv * (TKP / 128), nk = Hkv * (TKP / 64);
  const int blk = blockIdx.x;
  if (blk < nv) {
    const int g = blk % (TKP / 128), h = blk / (TKP / 128);
    const int seq = vk.ktab[g];
    if (seq < 0) return;
    const int kb = vk.cu_k[seq], n = vk.cu_k[seq + 1] - kb, local0 = g * 128 - vk.kp[seq];
    if (local0 >= n) return;  // padding only
    const float a = vamax_core<D, DT>(v + h * vsh + (int64_t)kb * vss, vss, local0, min(n, local0 + 128));
    if (threadIdx.x < HeadDim<D>::DP)
      atomicMax(reinterpret_cast<unsigned int*>(vs + ((int64_t)seq * Hkv + h) * HeadDim<D>::DP + threadIdx.x),
                __float_as_uint(a));
  } else if (blk < nv + nk) {
    const int i = blk - nv;
    const int g = i % (TKP / 64), h = i / (TKP / 64);
    const int seq = vk.ktab[g >> 1];
    if (seq < 0) return;
    const int kb = vk.cu_k[seq];
    quant_k64_core<D, DT>(k + h * ksh + (int64_t)kb * kss, kss, g * 64 - vk.kp[seq], vk.cu_k[seq + 1] - kb,
                          k8 + ((int64_t)h * TKP + g * 64) * HeadDim<D>::DP, ks + (int64_t)h * (TKP / SAGE_KV_BLOCK) + g * 2);
  } else {
    quant_q_rows<D, DT>(x, 0, qss, qsh, H, TQ, row_tiles, qs_mul, q8, qs, blk - nv - nk);
  }
}

// second launch: V of one padded 128-key block per workgroup, grid = Hkv * TKP / 128
template <int D, int DT>
__global__ __launch_bounds__(256) void quant_v_varlen_kernel(const uint16_t* __restrict__ v, int64_t vss, int64_t vsh,
                                                             int Hkv, int TKP, VarlenKeys vk,
                                                             const float* __restrict__ vs, uint8_t* __restrict__ v8t) {
  const int g = blockIdx.x % (TKP / 128), h = blockIdx.x / (TKP / 128);
  const int seq = vk.ktab[g];
  if (seq < 0) return;
  const int kb = vk.cu_k[seq];
  quant_v128_core<D, DT>(v + h * vsh + (int64_t)kb * vss, vss, g * 128 - vk.kp[seq], vk.cu_k[seq + 1] - kb,
                         vs + ((int64_t)seq * Hkv + h) * HeadDim<D>::DP, 0, nullptr,
                         v8t + (int64_t)h * HeadDim<D>::DP * TKP + g * 128, TKP);
}

// ------------------------------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------------------------------
static int check_common(int B, int H, int S, int D, int dtype, const char* who) {
  SAGE_REQUIRE(B > 0 && H > 0 && S > 0, "%s: sizes must be positive (B=%d H=%d S=%d)", who, B, H, S);
  if (!head_dim_ok(D)) return fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 96, 128, 256)", who, D);
  if (dtype != SAGE_DTYPE_BF16 && dtype != SAGE_DTYPE_F16)
    return fail(SAGE_ERR_UNSUPPORTED, "%s: dtype code %d (bf16=0, f16=1)", who, dtype);
  return SAGE_OK;
}

static int check_strided(const void* p, int64_t sb, int64_t ss, int64_t sh, const char* who, const char* name) {
  SAGE_REQUIRE(p != nullptr, "%s: %s is NULL", who, name);
  SAGE_REQUIRE(aligned16(p), "%s: %s is not 16-byte aligned", who, name);
  SAGE_REQUIRE(sb % 8 == 0 && ss % 8 == 0 && sh % 8 == 0 && sb >= 0 && ss >= 0 && sh >= 0,
               "%s: %s strides (%lld, %lld, %lld) must be non-negative multiples of 8 elements", who, name,
               (long long)sb, (long long)ss, (long long)sh);
  return SAGE_OK;
}

template <int D, int DT>
static void launch_quant_q(const void* q, int64_t sb, int64_t ss, int64_t sh, int B, int H, int S, float qs_mul,
                           int8_t* q8, float* qs, hipStream_t st) {
  const int tiles = (S + 63) / 64;
  hipLaunchKernelGGL((quant_q_kernel<D, DT>), dim3(tiles * B * H), dim3(256), 0, st,
                     static_cast<const uint16_t*>(q), sb, ss, sh, H, S, tiles, qs_mul, q8, qs);
}

template <int D, int DT>
static void launch_v_amax(const void* v, int64_t sb, int64_t ss, int64_t sh, int B, int Hkv, int S, float* vs,
                          hipStream_t st) {
  const int64_t n = (int64_t)B * Hkv * HeadDim<D>::DP;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, vs, n, 0.0f);
  // aim for ~256 rows per block, but keep the block count per (b, h) bounded
  int chunk_rows = 256;
  int chunks = (S + chunk_rows - 1) / chunk_rows;
  hipLaunchKernelGGL((v_amax_kernel<D, DT>), dim3(chunks * B * Hkv), dim3(256), 0, st, static_cast<const uint16_t*>(v),
                     sb, ss, sh, Hkv, S, chunks, chunk_rows, vs);
}

template <int D, int DT>
static void launch_quant_kv(const void* k, int64_t ksb, int64_t kss, int64_t ksh, const void* v, int64_t vsb,
                            int64_t vss, int64_t vsh, int B, int Hkv, int S, const float* vs, int8_t* k8, float* ks,
                            uint8_t* v8t, hipStream_t st) {
  const int Skp = kv_pad(S);
  hipLaunchKernelGGL((quant_kv_kernel<D, DT>), dim3(Skp / 128 * B * Hkv), dim3(256), 0, st,
                     static_cast<const uint16_t*>(k), ksb, kss, ksh, static_cast<const uint16_t*>(v), vsb, vss, vsh,
                     Hkv, S, Skp, vs, k8, ks, v8t);
}

// sage_forward's quantization in two launches: Q, K and per-chunk V maxima, then V (reducing the maxima).
template <int D, int DT>
static void launch_forward_quant(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb,
                                 int64_t kss, int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, int B,
                                 int H, int Hkv, int Sq, int Skv, float qs_mul, int8_t* q8, float* qs, float* vpart,
                                 int8_t* k8, float* ks, uint8_t* v8t, float* vs, const MaskPrep& mp, hipStream_t st) {
  const int tiles = (Sq + 63) / 64;
  const int Skp = kv_pad(Skv);
  const int vchunks = vamax_chunks(Skv);
  const int nv = vchunks * B * Hkv;
  const int nk = Skp / 64 * B * Hkv;
  const int nq = tiles * B * H;
  const int nvb = Skp / 128 * B * Hkv;
  hipLaunchKernelGGL((quant_qk_vamax_kernel<D, DT>), dim3(nv + nk + nq + mp.prep_blocks), dim3(256), 0, st,
                     static_cast<const uint16_t*>(q), qsb, qss, qsh, H, Sq, tiles, qs_mul, q8, qs,
                     static_cast<const uint16_t*>(k), ksb, kss, ksh, Skp, nk, k8, ks,
                     static_cast<const uint16_t*>(v), vsb, vss, vsh, Hkv, Skv, vchunks, nv, vpart, nq, mp);
  hipLaunchKernelGGL((quant_v_kernel<D, DT>), dim3(nvb + mp.range_blocks), dim3(256), 0, st,
                     static_cast<const uint16_t*>(v), vsb, vss, vsh, Hkv, Skv, Skp, vpart, vchunks, vs, v8t, nvb, mp);
}

template <int D, int DT>
static void launch_varlen_quant(const void* q, int64_t qss, int64_t qsh, const void* k, int64_t kss, int64_t ksh,
                                const void* v, int64_t vss, int64_t vsh, int H, int Hkv, int TQ, int TKP,
                                float qs_mul, VarlenKeys vk, int8_t* q8, float* qs, int8_t* k8, float* ks,
                                uint8_t* v8t, float* vs, hipStream_t st) {
  const int tiles = (TQ + 63) / 64;
  const int nv = Hkv * (TKP / 128), nk = Hkv * (TKP / 64);
  hipLaunchKernelGGL((quant_varlen_kernel<D, DT>), dim3(nv + nk + tiles * H), dim3(256), 0, st,
                     static_cast<const uint16_t*>(q), qss, qsh, H, TQ, tiles, qs_mul, q8, qs,
                     static_cast<const uint16_t*>(k), kss, ksh, static_cast<const uint16_t*>(v), vss, vsh, Hkv, TKP,
                     vk, k8, ks, vs);
  hipLaunchKernelGGL((quant_v_varlen_kernel<D, DT>), dim3(nv), dim3(256), 0, st, static_cast<const uint16_t*>(v),
                     vss, vsh, Hkv, TKP, vk, vs, v8t);
}

#define SAGE_DISPATCH_D_DT(D, DT, FN, ...)                                                   \
  do {                                                                                     \
    const bool bf_ = (DT) == SAGE_DTYPE_BF16;                                              \
    switch (D) {                                                                           \
      case 64: bf_ ? FN<64, DT_BF16>(__VA_ARGS__) : FN<64, DT_F16>(__VA_ARGS__); break;     \
      case 96: bf_ ? FN<96, DT_BF16>(__VA_ARGS__) : FN<96, DT_F16>(__VA_ARGS__); break;     \
      case 128: bf_ ? FN<128, DT_BF16>(__VA_ARGS__) : FN<128, DT_F16>(__VA_ARGS__); break;  \
      default: bf_ ? FN<256, DT_BF16>(__VA_ARGS__) : FN<256, DT_F16>(__VA_ARGS__); break;   \
    }                                                                                      \
  } while (0)

int quant_q_impl(const void* q, int64_t sb, int64_t ss, int64_t sh, int B, int H, int Sq, int D, int dtype,
                 float qs_mul, int8_t* q8, float* qs, void* stream) {
  const char* who = "sage_quant_q";
  int rc = check_common(B, H, Sq, D, dtype, who);
  if (rc) return rc;
  if ((rc = check_qs_mul(qs_mul, who))) return rc;
  if ((rc = check_strided(q, sb, ss, sh, who, "q"))) return rc;
  SAGE_REQUIRE(q8 != nullptr && qs != nullptr, "%s: q8 / qs is NULL", who);
  SAGE_REQUIRE(aligned16(q8), "%s: q8 is not 16-byte aligned", who);
  SAGE_DISPATCH_D_DT(D, dtype, launch_quant_q, q, sb, ss, sh, B, H, Sq, qs_mul, q8, qs, (hipStream_t)stream);
  return check_launch("quant_q launch");
}

int v_amax_impl(const void* v, int64_t sb, int64_t ss, int64_t sh, int B, int Hkv, int Skv, int D, int dtype,
                float* vs, void* stream) {
  const char* who = "sage_v_amax";
  int rc = check_common(B, Hkv, Skv, D, dtype, who);
  if (rc) return rc;
  if ((rc = check_strided(v, sb, ss, sh, who, "v"))) return rc;
  SAGE_REQUIRE(vs != nullptr, "%s: vs is NULL", who);
  SAGE_DISPATCH_D_DT(D, dtype, launch_v_amax, v, sb, ss, sh, B, Hkv, Skv, vs, (hipStream_t)stream);
  return check_launch("v_amax launch");
}

int quant_kv_impl(const void* k, int64_t ksb, int64_t kss, int64_t ksh, const void* v, int64_t vsb, int64_t vss,
                  int64_t vsh, int B, int Hkv, int Skv, int D, int dtype, const float* vs, int8_t* k8, float* ks,
                  uint8_t* v8t, void* stream) {
  const char* who = "sage_quant_kv";
  int rc = check_common(B, Hkv, Skv, D, dtype, who);
  if (rc) return rc;
  if ((rc = check_strided(k, ksb, kss, ksh, who, "k"))) return rc;
  if ((rc = check_strided(v, vsb, vss, vsh, who, "v"))) return rc;
  SAGE_REQUIRE(vs != nullptr && k8 != nullptr && ks != nullptr && v8t != nullptr, "%s: an output pointer is NULL", who);
  SAGE_REQUIRE(aligned16(k8) && aligned16(v8t), "%s: k8 / v8t must be 16-byte aligned", who);
  SAGE_DISPATCH_D_DT(D, dtype, launch_quant_kv, k, ksb, kss, ksh, v, vsb, vss, vsh, B, Hkv, Skv, vs, k8, ks, v8t,
                     (hipStream_t)stream);
  return check_launch("quant_kv launch");
}

int64_t vamax_partial_bytes(int B, int Hkv, int Skv, int D) {
  return (int64_t)B * Hkv * vamax_chunks(Skv) * layout_dim(D) * (int64_t)sizeof(float);
}

// sage_forward's inputs, checked before its first launch (sizes, dtype, head dim, pointers and strides of q, k, v).
int forward_inputs_check(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                         int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, int B, int H, int Hkv,
                         int Sq, int Skv, int D, int dtype, const char* who) {
  int rc = check_common(B, H, Sq, D, dtype, who);
  if (rc) return rc;
  if ((rc = check_common(B, Hkv, Skv, D, dtype, who))) return rc;
  if ((rc = check_strided(q, qsb, qss, qsh, who, "q"))) return rc;
  if ((rc = check_strided(k, ksb, kss, ksh, who, "k"))) return rc;
  return check_strided(v, vsb, vss, vsh, who, "v");
}

// Validation of every argument is done by the caller (sage_forward) through the per-stage checks below.  mp: the
// mask work of sage_forward_masked (NULL: none), run as extra workgroups of the two launches.
int forward_quant_impl(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                       int64_t ksh, const void* v, int64_t vsb, int64_t vss, int64_t vsh, int B, int H, int Hkv, int Sq,
                       int Skv, int D, int dtype, float qs_mul, int8_t* q8, float* qs, float* vpart, int8_t* k8,
                       float* ks, uint8_t* v8t, float* vs, const MaskPrep* mp, void* stream) {
  const char* who = "sage_forward";
  int rc = forward_inputs_check(q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, B, H, Hkv, Sq, Skv, D, dtype, who);
  if (rc) return rc;
  SAGE_REQUIRE(q8 && qs && vpart && k8 && ks && v8t && vs, "%s: an intermediate pointer is NULL", who);
  SAGE_REQUIRE(aligned16(q8) && aligned16(k8) && aligned16(v8t) && aligned16(vpart) && aligned16(vs),
               "%s: q8 / k8 / v8t / vs / workspace must be 16-byte aligned", who);
  const MaskPrep none{};
  SAGE_DISPATCH_D_DT(D, dtype, launch_forward_quant, q, qsb, qss, qsh, k, ksb, kss, ksh, v, vsb, vss, vsh, B, H, Hkv,
                     Sq, Skv, qs_mul, q8, qs, vpart, k8, ks, v8t, vs, mp ? *mp : none, (hipStream_t)stream);
  return check_launch("quantization launch");
}

// Validation is done by the caller (sage_forward_varlen); vs must already be zero.
int varlen_quant_impl(const void* q, int64_t qss, int64_t qsh, const void* k, int64_t kss, int64_t ksh, const void* v,
                      int64_t vss, int64_t vsh, int H, int Hkv, int TQ, int TKP, int D, int dtype, float qs_mul,
                      const int* cu_k, const int* kp, const int* ktab, int8_t* q8, float* qs, int8_t* k8, float* ks,
                      uint8_t* v8t, float* vs, void* stream) {
  const VarlenKeys vk{cu_k, kp, ktab};
  SAGE_DISPATCH_D_DT(D, dtype, launch_varlen_quant, q, qss, qsh, k, kss, ksh, v, vss, vsh, H, Hkv, TQ, TKP, qs_mul, vk,
                     q8, qs, k8, ks, v8t, vs, (hipStream_t)stream);
  return check_launch("varlen quantization launch");
}

}  // namespace sage

extern "C" int sage_quant_q(const void* q, int64_t sb, int64_t ss, int64_t sh, int B, int H, int Sq, int D, int dtype,
                            float qs_mul, int8_t* q8, float* qs, void* stream) {
  sage::clear_error();
  return sage::quant_q_impl(q, sb, ss, sh, B, H, Sq, D, dtype, qs_mul, q8, qs, stream);
}

extern "C" int sage_v_amax(const void* v, int64_t sb, int64_t ss, int64_t sh, int B, int Hkv, int Skv, int D, int dtype,
                           float* vs, void* stream) {
  sage::clear_error();
  return sage::v_amax_impl(v, sb, ss, sh, B, Hkv, Skv, D, dtype, vs, stream);
}

extern "C" int sage_quant_kv(const void* k, int64_t ksb, int64_t kss, int64_t ksh, const void* v, int64_t vsb,
                             int64_t vss, int64_t vsh, int B, int Hkv, int Skv, int D, int dtype, const float* vs,
                             int8_t* k8, float* ks, uint8_t* v8t, void* stream) {
  sage::clear_error();
  return sage::quant_kv_impl(k, ksb, kss, ksh, v, vsb, vss, vsh, B, Hkv, Skv, D, dtype, vs, k8, ks, v8t, stream);
}
