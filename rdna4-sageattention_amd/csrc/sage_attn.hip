// int8 QK^T / fp8 PV flash attention for gfx950 (CDNA4, wave64 MFMA).
//
// Math (the reference kernel's, kernel_build/make_sage.py:75-107, :196-237; make_sage_r2.py:54-269):
//   cl_i   = fp32(sm * log2e) * QS_i                      (sm = 1/sqrt(D) baked in; other scales folded into QS)
//   S_ij   = sum_d Q8_id K8_jd                            (int32, exact)
//   rowmax = max over the tile's 32-key blocks of (max_j S_ij) * KS_block
//   lazy rescale: m_cand = max(m, rowmax); need = (m_cand - m) * cl > 8; m_new = need ? m_cand : m
//   p_ij   = exp2(fma(S_ij, cl * KS_block, -(cl * m_new)))   (<= 2^8, fits E4M3)
//   l      = corr * l + sum_j p_ij (fp32 p);  O = need ? O * corr : O;  O += e4m3(p) V8
//   out    = (O * ((1/448) / l)) * VS
//
// gfx950 mapping.  A workgroup owns 128 query rows (4 waves x 32) of one (batch, head) and walks the KV sequence
// in 64-key tiles staged in LDS (double buffered; the next tile's global loads are in flight while the current
// one is computed).  Per wave and tile:
//   * S^T = K Q^T with v_mfma_i32_32x32x32_i8: A = 32 keys x 32 dims of K (LDS), B = 32 dims x 32 queries of Q
//     (registers for the whole kernel).  The 32x32 accumulator gives lane l the query l % 32 and 16 keys
//     8(v/4) + 4(l/32) + v%4 of the block (v = accumulator register), so row statistics need one exchange with lane
//     l ^ 32 and no other cross-lane traffic.
//   * The 2 x 16 probabilities of a lane, cast to E4M3 in register order, are exactly the lane's 32-byte B operand
//     of v_mfma_f32_32x32x64_f8f6f4 for O^T = V^T P^T: B = 64 keys x 32 queries.  The A operand (32 channels x 64
//     keys of V) must hold the same keys in the same byte order; the quantizer stores V8T with keys permuted inside
//     each 64-key group (key 8g + 4h + r at position 32h + 4g + r), so each lane's A operand is 32 contiguous bytes.
//   * O^T accumulators (D/32 blocks of 32 channels) give lane l the same query as its S values: m, l and the
//     rescale stay per lane.
// LDS tiles use a 16-byte-chunk XOR swizzle so the MFMA operand reads are free of bank conflicts.
#include "sage_common.h"
#include "sage_host.h"

namespace sage {

constexpr int ATT_BM = 128;  // query rows per workgroup
constexpr int ATT_BN = 64;   // keys per tile
constexpr int ATT_THREADS = 256;

// chunk swizzle for LDS rows of `row_bytes` (64 or 128)
template <int ROW_BYTES> __device__ __forceinline__ int swz(int row, int chunk) {
  if (ROW_BYTES == 128) return chunk ^ ((row >> 1) & 7);
  return chunk ^ ((row >> 2) & 3);
}

template <int D, bool CAUSAL, int OUT_DT>
__global__ __launch_bounds__(ATT_THREADS, 2) void attn_kernel(
    const int8_t* __restrict__ q8, const float* __restrict__ qs, const int8_t* __restrict__ k8,
    const float* __restrict__ ks, const uint8_t* __restrict__ v8t, const float* __restrict__ vs,
    uint16_t* __restrict__ out, int64_t osb, int64_t oss, int64_t osh, float* __restrict__ lse, int H, int Hkv,
    int Sq, int Skv, int Skp, int q_tiles, int total, float c0) {
  constexpr int BN = ATT_BN;
  constexpr int KTILE = BN * D;      // bytes of the K tile  ([64 keys][D])
  constexpr int VTILE = D * BN;      // bytes of the V tile  ([D channels][64 keys])
  constexpr int NQK = D / 32;        // i8 MFMAs (K = 32 dims) per 32-key block
  constexpr int NPV = D / 32;        // fp8 MFMAs (M = 32 channels) per tile
  constexpr int KCH = D / 16;        // 16-byte chunks per K row
  constexpr int NKL = KTILE / 16 / ATT_THREADS;  // K chunks per thread per tile
  constexpr int NVL = VTILE / 16 / ATT_THREADS;  // V chunks per thread per tile
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][KTILE + VTILE];

  // ---- work decode ----
  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / q_tiles;
  int qt = logical % q_tiles;
  if (CAUSAL) qt = q_tiles - 1 - qt;  // longest rows first within a head
  const int b = bh / H, h = bh % H;
  const int hkv = h / (H / Hkv);
  const int bhk = b * Hkv + hkv;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, hf = lane >> 5;
  const int q0 = qt * ATT_BM + wave * 32;
  const int qrow = q0 + ln;
  const bool qvalid = qrow < Sq;
  const int qr = qvalid ? qrow : Sq - 1;
  const int off = Skv - Sq;  // bottom-right causal offset

  // ---- Q operand (B of the QK MFMA): lane (query ln, half hf) holds dims [32i + 16hf, +16) ----
  v4i qa[NQK];
  {
    const int8_t* qp = q8 + ((int64_t)bh * Sq + qr) * D + 16 * hf;
#pragma unroll
    for (int i = 0; i < NQK; ++i) qa[i] = *reinterpret_cast<const v4i*>(qp + 32 * i);
  }
  const float cl = c0 * qs[(int64_t)bh * Sq + qr];

  // ---- KV range ----
  int kv_end = Skv;
  if (CAUSAL) kv_end = min(Skv, qt * ATT_BM + ATT_BM + off);
  const int ntiles = (kv_end + BN - 1) / BN;
  const int wave_last_key = CAUSAL ? min(Skv - 1, q0 + 31 + off) : Skv - 1;

  const int8_t* kbase = k8 + (int64_t)bhk * Skp * D;
  const uint8_t* vbase = v8t + (int64_t)bhk * D * Skp;
  const float* ksb = ks + (int64_t)bhk * (Skp / SAGE_KV_BLOCK);

  uint4 kreg[NKL], vreg[NVL];
  auto load_tile = [&](int t) {
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
      const int c = tid + i * ATT_THREADS;
      kreg[i] = *reinterpret_cast<const uint4*>(kbase + (int64_t)t * KTILE + c * 16);
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      const int c = tid + i * ATT_THREADS;
      const int d = c >> 2, col = c & 3;
      vreg[i] = *reinterpret_cast<const uint4*>(vbase + (int64_t)d * Skp + t * BN + col * 16);
    }
  };
  auto store_tile = [&](int buf) {
    uint8_t* kt = smem[buf];
    uint8_t* vt = smem[buf] + KTILE;
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
      const int c = tid + i * ATT_THREADS;
      const int row = c / KCH, col = c % KCH;
      *reinterpret_cast<uint4*>(kt + row * D + swz<D>(row, col) * 16) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      const int c = tid + i * ATT_THREADS;
      const int d = c >> 2, col = c & 3;
      *reinterpret_cast<uint4*>(vt + d * BN + swz<BN>(d, col) * 16) = vreg[i];
    }
  };

  v16f o[NPV];
#pragma unroll
  for (int i = 0; i < NPV; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[i][v] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);
    const int kstart = t * BN;
    if (kstart <= wave_last_key) {
      const uint8_t* kt = smem[buf];
      const uint8_t* vt = smem[buf] + KTILE;
      // ---- S^T = K Q^T ----
      v16i s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) s[kb][v] = 0;
        const int row = 32 * kb + ln;
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
          const v4i ka = *reinterpret_cast<const v4i*>(kt + row * D + swz<D>(row, 2 * i + hf) * 16);
          s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, qa[i], s[kb], 0, 0, 0);
        }
      }
      // ---- online softmax ----
      float sf[2][16];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) sf[kb][v] = (float)s[kb][v];
      const bool need_mask = (kstart + BN > Skv) || (CAUSAL && kstart + BN - 1 > q0 + off);
      if (need_mask) {
        const int last = qr + off;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = kstart + 32 * kb + 8 * (v >> 2) + 4 * hf + (v & 3);
            if (key >= Skv || (CAUSAL && key > last)) sf[kb][v] = -INFINITY;
          }
      }
      float mx0 = sf[0][0], mx1 = sf[1][0];
#pragma unroll
      for (int v = 1; v < 16; ++v) {
        mx0 = fmaxf(mx0, sf[0][v]);
        mx1 = fmaxf(mx1, sf[1][v]);
      }
      mx0 = fmaxf(mx0, xor32_f32(mx0));
      mx1 = fmaxf(mx1, xor32_f32(mx1));
      const float ks0 = ksb[2 * t], ks1 = ksb[2 * t + 1];
      const float rowmax = fmaxf(mx0 * ks0, mx1 * ks1);
      const float m_cand = fmaxf(m, rowmax);
      const bool need = (m_cand - m) * cl > 8.0f;
      const float m_new = need ? m_cand : m;
      const float corr = __builtin_amdgcn_exp2f((m - m_new) * cl);
      const float neg = 0.0f - cl * m_new;
      const float ct0 = cl * ks0, ct1 = cl * ks1;
      float p[2][16];
      float psum = 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        p[0][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sf[0][v], ct0, neg));
        psum += p[0][v];
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        p[1][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sf[1][v], ct1, neg));
        psum += p[1][v];
      }
      l = corr * l + psum;
      m = m_new;
      if (__builtin_amdgcn_read_exec() & __ballot(need)) {
#pragma unroll
        for (int i = 0; i < NPV; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[i][v] *= corr;
      }
      // ---- P -> E4M3, B operand byte t = 16 kb + v ----
      v8i pb;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const int kb = w >> 2, v0 = 4 * (w & 3);
        int d = 0;
        d = __builtin_amdgcn_cvt_pk_fp8_f32(p[kb][v0], p[kb][v0 + 1], d, false);
        d = __builtin_amdgcn_cvt_pk_fp8_f32(p[kb][v0 + 2], p[kb][v0 + 3], d, true);
        pb[w] = d;
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        const int d = 32 * i + ln;
        const v4i a0 = *reinterpret_cast<const v4i*>(vt + d * BN + swz<BN>(d, 2 * hf) * 16);
        const v4i a1 = *reinterpret_cast<const v4i*>(vt + d * BN + swz<BN>(d, 2 * hf + 1) * 16);
        const v8i va = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        o[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va, pb, o[i], 0, 0, 0, 0, 0, 0);
      }
    }
    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const float lt = l + xor32_f32(l);
  const float inv = (1.0f / 448.0f) / lt;
  if (qvalid) {
    uint16_t* orow = out + b * osb + (int64_t)qrow * oss + h * osh;
    const float* vsr = vs + (int64_t)bhk * D;
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = 32 * i + 8 * g + 4 * hf;
        const v4f sc = *reinterpret_cast<const v4f*>(vsr + c);
        const uint32_t e0 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 0] * inv) * sc[0]);
        const uint32_t e1 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 1] * inv) * sc[1]);
        const uint32_t e2 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 2] * inv) * sc[2]);
        const uint32_t e3 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 3] * inv) * sc[3]);
        *reinterpret_cast<uint2*>(orow + c) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
      }
    }
    if (lse != nullptr && hf == 0) {
      // sum_j exp(logit_ij) = 2^(cl * m) * l_total, so lse = ln2 * (cl * m + log2(l_total))
      lse[(int64_t)bh * Sq + qrow] = 0.69314718055994531f * (cl * m + __log2f(lt));
    }
  }
}

template <int D, bool CAUSAL, int OUT_DT>
static void launch_attn(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                        const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, float* lse, int B, int H,
                        int Hkv, int Sq, int Skv, hipStream_t st) {
  const int q_tiles = (Sq + ATT_BM - 1) / ATT_BM;
  const int total = B * H * q_tiles;
  const float c0 = (float)((1.0 / __builtin_sqrt((double)D)) * 1.4426950408889634);
  hipLaunchKernelGGL((attn_kernel<D, CAUSAL, OUT_DT>), dim3(total), dim3(ATT_THREADS), 0, st, q8, qs, k8, ks, v8t, vs,
                     static_cast<uint16_t*>(out), osb, oss, osh, lse, H, Hkv, Sq, Skv, kv_pad(Skv), q_tiles, total, c0);
}

int attn_impl(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t, const float* vs,
              void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D,
              int causal, int out_dtype, float* lse, void* stream) {
  const char* who = "sage_attn_fwd";
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "%s: sizes must be positive", who);
  SAGE_REQUIRE(H % Hkv == 0, "%s: heads %d not a multiple of kv heads %d", who, H, Hkv);
  if (D != 64 && D != 128) return fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 128)", who, D);
  if (out_dtype != SAGE_DTYPE_BF16 && out_dtype != SAGE_DTYPE_F16)
    return fail(SAGE_ERR_UNSUPPORTED, "%s: out dtype code %d", who, out_dtype);
  if (causal && Sq != Skv) return fail(SAGE_ERR_UNSUPPORTED, "%s: causal attention needs q_len == kv_len", who);
  SAGE_REQUIRE(q8 && qs && k8 && ks && v8t && vs && out, "%s: a pointer argument is NULL", who);
  SAGE_REQUIRE(aligned16(q8) && aligned16(k8) && aligned16(v8t) && aligned16(vs) && aligned16(out),
               "%s: q8 / k8 / v8t / vs / out must be 16-byte aligned", who);
  SAGE_REQUIRE(osb % 8 == 0 && oss % 8 == 0 && osh % 8 == 0 && osb >= 0 && oss >= 0 && osh >= 0,
               "%s: out strides must be non-negative multiples of 8 elements", who);
  SAGE_REQUIRE((int64_t)B * H * ((Sq + ATT_BM - 1) / ATT_BM) < (1ll << 31), "%s: too many query tiles", who);
  hipStream_t st = (hipStream_t)stream;
#define SAGE_ATTN_CASE(DD, CC, OO) \
  launch_attn<DD, CC, OO>(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, lse, B, H, Hkv, Sq, Skv, st)
  const bool bf = out_dtype == SAGE_DTYPE_BF16;
  if (D == 128) {
    if (causal) { if (bf) SAGE_ATTN_CASE(128, true, DT_BF16); else SAGE_ATTN_CASE(128, true, DT_F16); }
    else { if (bf) SAGE_ATTN_CASE(128, false, DT_BF16); else SAGE_ATTN_CASE(128, false, DT_F16); }
  } else {
    if (causal) { if (bf) SAGE_ATTN_CASE(64, true, DT_BF16); else SAGE_ATTN_CASE(64, true, DT_F16); }
    else { if (bf) SAGE_ATTN_CASE(64, false, DT_BF16); else SAGE_ATTN_CASE(64, false, DT_F16); }
  }
#undef SAGE_ATTN_CASE
  return check_launch("attention launch");
}

}  // namespace sage

extern "C" int sage_attn_fwd(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                             const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv,
                             int Sq, int Skv, int D, int causal, int out_dtype, float* lse, void* stream) {
  sage::clear_error();
  return sage::attn_impl(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, causal, out_dtype, lse,
                         stream);
}
