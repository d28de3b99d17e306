// Row logsumexp of (Q K^T) * sm_scale over the keys, natural log, fp32 [B, H, Sq], on the bf16 / fp16 inputs
// (what `return_lse` returns; reference: src/sageattention/core.py:23-44, an fp32 torch matmul plus logsumexp per row
// chunk).  Products of two 16-bit floats are exact in fp32, so the MFMA's fp32 accumulation gives the scores to fp32
// accuracy, as the reference's fp32 matmul does.
//
// gfx950 mapping: a workgroup owns 128 query rows (4 waves x 32) of one (batch, head) and walks the keys in 64-key tiles
// copied global -> LDS (direct loads, double buffered, 16-byte chunks XOR-swizzled by row; the tiles no row of a
// wave needs masked run a mask-free body).  Per wave and tile,
// S^T = K Q^T with v_mfma_f32_32x32x16_{bf16,f16}: A = 32 keys x 16 dims of K from LDS, B = Q from registers.  The
// accumulator gives lane l the query l % 32 and 16 keys of each 32-key block, so the row statistics need one exchange
// with lane l ^ 32.  Statistics are an online max / sum in the log2 domain: l = sum_j 2^((s_ij - m) * c) with
// c = sm_scale * log2(e) and lse = ln 2 * (m * c + log2 l), for any m that keeps the terms finite.  m is the running
// max, raised only when needed: once every row of a wave has one, a tile first adds its terms with the current m and
// keeps them when every lane's sum is below 2^16 (almost always; an overflow gives inf and fails the test), else it
// takes the tile's max as the exact online update does.  Causal masks are bottom-right aligned (Sq <= Skv).
#include <type_traits>

#include "sage_common.h"
#include "sage_host.h"

namespace sage {

constexpr int LSE_BM = 128;  // query rows per workgroup
constexpr int LSE_BN = 64;   // keys per tile
constexpr int LSE_THREADS = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int DT> __device__ __forceinline__ v16f mfma_32x32x16(v4i a, v4i b, v16f c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

// 16-byte chunk c of LDS row `row` (rows of KCH chunks): conflict-free MFMA operand reads for 32 consecutive rows
template <int KCH> __device__ __forceinline__ int lse_swz(int row, int c) { return c ^ (row & (KCH - 1)); }

__device__ __forceinline__ void lse_copy16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <int D, bool CAUSAL, int DT>
__global__ __launch_bounds__(LSE_THREADS, 2) void lse_kernel(const uint16_t* __restrict__ q, int64_t qsb, int64_t qss,
                                                             int64_t qsh, const uint16_t* __restrict__ k, int64_t ksb,
                                                             int64_t kss, int64_t ksh, int H, int Hkv, int Sq,
                                                             int Skv, int q_tiles, int total, float c,
                                                             float* __restrict__ lse) {
  constexpr int BN = LSE_BN;
  constexpr int ROWB = D * 2;              // bytes per K row
  constexpr int KCH = ROWB / 16;           // 16-byte chunks per row
  constexpr int KTILE = BN * ROWB;         // bytes per K tile
  constexpr int NK = D / 16;               // MFMAs (16 dims each) per 32-key block
  constexpr int LOADS = KTILE / 1024 / 4;  // 1 KiB direct loads per wave per tile
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][KTILE];

  int bh, qt;
  if (CAUSAL) {
    causal_tile(blockIdx.x, total / q_tiles, q_tiles, bh, qt);
  } else {
    const int logical = xcd_remap(blockIdx.x, total);
    bh = logical / q_tiles;
    qt = logical % q_tiles;
  }
  const int b = bh / H, h = bh % H;
  const int hkv = h / (H / Hkv);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, hf = lane >> 5;
  const int q0 = qt * LSE_BM + wave * 32;
  const int qrow = q0 + ln;
  const bool qvalid = qrow < Sq;
  const int qr = qvalid ? qrow : Sq - 1;
  const int off = Skv - Sq;  // bottom-right causal offset (>= 0)

  // Q operand (B of the MFMA): lane (query ln, half hf) holds dims [16 i + 8 hf, +8)
  v4i qa[NK];
  {
    const uint16_t* qp = q + b * qsb + (int64_t)qr * qss + h * qsh + 8 * hf;
#pragma unroll
    for (int i = 0; i < NK; ++i) qa[i] = *reinterpret_cast<const v4i*>(qp + 16 * i);
  }

  int kv_end = Skv;
  if (CAUSAL) kv_end = min(Skv, qt * LSE_BM + LSE_BM + off);
  const int ntiles = (kv_end + BN - 1) / BN;
  const uint16_t* kbase = k + b * ksb + hkv * ksh;

  // direct-load sources: load j of wave w fills LDS chunk L = (w * LOADS + j) * 64 + lane, which holds tile row
  // L / KCH, logical chunk lse_swz(row, L % KCH) (the swizzle is an involution)
  int lrow[LOADS], lchunk[LOADS];
  uint32_t koff[LOADS];  // byte offset of the load inside a whole tile (64 * kss < 2^31, checked on the host)
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int L = (wave * LOADS + j) * 64 + lane;
    lrow[j] = L / KCH;
    lchunk[j] = lse_swz<KCH>(lrow[j], L % KCH) * 8;  // in elements
    koff[j] = (uint32_t)(((int64_t)lrow[j] * kss + lchunk[j]) * 2);
  }
  // Whole tiles: the tile base pinned to an SGPR pair plus the lane's 32-bit offset (the saddr + voffset form, no
  // per-load 64-bit address arithmetic).  The last tile, when partial, repeats the last key in its rows past Skv
  // (masked below).
  auto issue = [&](int t, int buf) {
    uint8_t* dst = smem[buf];
    if ((t + 1) * BN <= Skv) {
      const uint8_t* kb = reinterpret_cast<const uint8_t*>(kbase + (int64_t)t * BN * kss);
      asm volatile("" : "+s"(kb));
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        asm volatile("" : "+v"(koff[j]));
        lse_copy16(kb + koff[j], dst + (wave * LOADS + j) * 1024);
      }
    } else {
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        const int key = min(t * BN + lrow[j], Skv - 1);
        lse_copy16(kbase + (int64_t)key * kss + lchunk[j], dst + (wave * LOADS + j) * 1024);
      }
    }
  };

  int ko[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) ko[i] = ln * ROWB + lse_swz<KCH>(ln, 2 * i + hf) * 16;

  float m = -INFINITY, l = 0.0f;
  float negm = 0.0f;    // -(m * c) once m is finite
  bool fastok = false;  // every row of the wave has a finite m: tiles start with the current m
  // One tile: S^T from the LDS buffer, the MASKED body clears keys past Skv and (causal) past the row's diagonal.
  // The two bodies sit in two loops (tiles before t_mask need no mask for any row of the wave): with the mask test
  // in one loop the compiler turns the masking into compares and selects on every tile.
  auto tile = [&](int t, auto masked, auto buf) {
    constexpr bool MASKED = decltype(masked)::value;
    const uint8_t* kt = smem[buf];  // a compile-time buffer in the mask-free loop: the LDS reads take it as an offset
    v16f s0 = {}, s1 = {};
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const v4i a0 = *reinterpret_cast<const v4i*>(kt + ko[i]);
      const v4i a1 = *reinterpret_cast<const v4i*>(kt + ko[i] + 32 * ROWB);
      s0 = mfma_32x32x16<DT>(a0, qa[i], s0);
      s1 = mfma_32x32x16<DT>(a1, qa[i], s1);
    }
    float sv[2][16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      sv[0][v] = s0[v];
      sv[1][v] = s1[v];
    }
    if constexpr (MASKED) {
      // element (kb, v) holds key t * 64 + 4 hf + (32 kb + 8 (v / 4) + v % 4): visible iff that offset <= lim
      const int lim = (CAUSAL ? min(Skv - 1, qr + off) : Skv - 1) - (t * BN + 4 * hf);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (32 * kb + 8 * (v >> 2) + (v & 3) > lim) sv[kb][v] = -INFINITY;
    }
    bool exact = !fastok;
    if (fastok) {
      float ps[4];  // four chains, each starting from its first term (0 + p is p: exp2 never gives -0)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[kb][v], c, negm));
          ps[v & 3] = (kb == 0 && v < 4) ? e : ps[v & 3] + e;
        }
      const float tsum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
      exact = __ballot(!(tsum < 65536.0f)) != 0;
      if (!exact) l = l + tsum;
    }
    if (exact) {
      float mx = sv[0][0];
#pragma unroll
      for (int v = 1; v < 16; ++v) mx = fmaxf(mx, sv[0][v]);
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sv[1][v]);
      mx = max_xor32_f32(mx);
      const float m_new = fmaxf(m, mx);
      const float corr = __builtin_amdgcn_exp2f((m - m_new) * c);  // m = -inf on the first tile: corr = 0
      const float neg = 0.0f - m_new * c;
      float ps[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[kb][v], c, neg));
          ps[v & 3] = (kb == 0 && v < 4) ? e : ps[v & 3] + e;
        }
      l = l * corr + ((ps[0] + ps[1]) + (ps[2] + ps[3]));
      m = m_new;
      negm = m == -INFINITY ? 0.0f : neg;  // a row with no visible key yet keeps m = -inf
      fastok = __ballot(m == -INFINITY) == 0;
    }
    // the wait for the next tile's direct loads comes after this tile's arithmetic (l is its last result; without
    // the operand the scheduler may hoist the wait into the middle of the tile)
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(l) : : "memory");
    __syncthreads();
  };
  // tiles before t_mask end below Skv and (causal) at or before the wave's first row's diagonal
  int t_mask = Skv / BN;
  if (CAUSAL) t_mask = min(t_mask, max(0, (q0 + off + 1) / BN));
  t_mask = min(t_mask, ntiles);
  issue(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int t = 0;
  // the mask-free tiles in pairs (t even: buffer 0, then 1), so that each body's buffer is a constant
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  for (; t + 1 < t_mask; t += 2) {
    issue(t + 1, 1);
    tile(t, std::false_type{}, B0{});
    if (t + 2 < ntiles) issue(t + 2, 0);
    tile(t + 1, std::false_type{}, B1{});
  }
  if (t < t_mask) {
    if (t + 1 < ntiles) issue(t + 1, 1);
    tile(t, std::false_type{}, B0{});
    ++t;
  }
  for (; t < ntiles; ++t) {
    if (t + 1 < ntiles) issue(t + 1, (t + 1) & 1);
    tile(t, std::true_type{}, t & 1);
  }
  const float lt = add_xor32_f32(l);
  if (qvalid && hf == 0) lse[(int64_t)bh * Sq + qrow] = 0.69314718055994531f * (m * c + __log2f(lt));
}

template <int D, bool CAUSAL, int DT>
static void launch_lse(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
                       int64_t ksh, int B, int H, int Hkv, int Sq, int Skv, float c, float* lse, hipStream_t st) {
  const int q_tiles = (Sq + LSE_BM - 1) / LSE_BM;
  const int total = B * H * q_tiles;
  hipLaunchKernelGGL((lse_kernel<D, CAUSAL, DT>), dim3(total), dim3(LSE_THREADS), 0, st,
                     static_cast<const uint16_t*>(q), qsb, qss, qsh, static_cast<const uint16_t*>(k), ksb, kss, ksh, H,
                     Hkv, Sq, Skv, q_tiles, total, c, lse);
}

int lse_impl(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb, int64_t kss,
             int64_t ksh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype, int causal, float sm_scale,
             float* lse, void* stream) {
  const char* who = "sage_lse_fwd";
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "%s: sizes must be positive", who);
  SAGE_REQUIRE(H % Hkv == 0, "%s: heads %d not a multiple of kv heads %d", who, H, Hkv);
  if (D != 64 && D != 128) return fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 128)", who, D);
  if (dtype != SAGE_DTYPE_BF16 && dtype != SAGE_DTYPE_F16)
    return fail(SAGE_ERR_UNSUPPORTED, "%s: dtype code %d (bf16=0, f16=1)", who, dtype);
  if (causal && Sq > Skv) return fail(SAGE_ERR_UNSUPPORTED, "%s: causal LSE needs q_len <= kv_len", who);
  SAGE_REQUIRE(q && k && lse, "%s: a pointer argument is NULL", who);
  SAGE_REQUIRE(aligned16(q) && aligned16(k), "%s: q / k must be 16-byte aligned", who);
  SAGE_REQUIRE(qsb % 8 == 0 && qss % 8 == 0 && qsh % 8 == 0 && ksb % 8 == 0 && kss % 8 == 0 && ksh % 8 == 0 &&
                   qsb >= 0 && qss >= 0 && qsh >= 0 && ksb >= 0 && kss >= 0 && ksh >= 0,
               "%s: strides must be non-negative multiples of 8 elements", who);
  SAGE_REQUIRE((int64_t)B * H * ((Sq + LSE_BM - 1) / LSE_BM) < (1ll << 31), "%s: too many query tiles", who);
  SAGE_REQUIRE((int64_t)LSE_BN * kss < (1ll << 31), "%s: key stride too large", who);
  const double scale = sm_scale > 0.0f ? (double)sm_scale : 1.0 / __builtin_sqrt((double)D);
  const float c = (float)(scale * 1.4426950408889634);
  hipStream_t st = (hipStream_t)stream;
#define SAGE_LSE_CASE(DD, CC, TT) \
  launch_lse<DD, CC, TT>(q, qsb, qss, qsh, k, ksb, kss, ksh, B, H, Hkv, Sq, Skv, c, lse, st)
  const bool bf = dtype == SAGE_DTYPE_BF16;
  if (D == 128) {
    if (causal) { if (bf) SAGE_LSE_CASE(128, true, DT_BF16); else SAGE_LSE_CASE(128, true, DT_F16); }
    else { if (bf) SAGE_LSE_CASE(128, false, DT_BF16); else SAGE_LSE_CASE(128, false, DT_F16); }
  } else {
    if (causal) { if (bf) SAGE_LSE_CASE(64, true, DT_BF16); else SAGE_LSE_CASE(64, true, DT_F16); }
    else { if (bf) SAGE_LSE_CASE(64, false, DT_BF16); else SAGE_LSE_CASE(64, false, DT_F16); }
  }
#undef SAGE_LSE_CASE
  return check_launch("lse launch");
}

}  // namespace sage

extern "C" int sage_lse_fwd(const void* q, int64_t qsb, int64_t qss, int64_t qsh, const void* k, int64_t ksb,
                            int64_t kss, int64_t ksh, int B, int H, int Hkv, int Sq, int Skv, int D, int dtype,
                            int causal, float sm_scale, float* lse, void* stream) {
  sage::clear_error();
  return sage::lse_impl(q, qsb, qss, qsh, k, ksb, kss, ksh, B, H, Hkv, Sq, Skv, D, dtype, causal, sm_scale, lse, stream);
}
