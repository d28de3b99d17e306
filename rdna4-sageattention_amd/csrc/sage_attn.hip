// int8 QK^T / fp8 PV flash attention for gfx950 (CDNA4, wave64 MFMA).
//
// Math (the reference kernel's: kernel_build/make_sage.py:75-107, :196-237; make_sage_r2.py:52-269, 32-key tiles
// per kernel_build/compile_attn.py:19):
//   cl_i   = fp32(sm * log2e) * QS_i                      (sm = 1/sqrt(D) baked in; other scales folded into QS)
//   S_ij   = sum_d Q8_id K8_jd                            (int32, exact; |S| <= 127^2 * D)
//   per 32-key block (one K scale KS_block each, make_sage_r2.py:141-190):
//     rowmax = (max_j S_ij) * KS_block
//     lazy rescale: m_cand = max(m, rowmax); need = (m_cand - m) * cl > 8; m_new = need ? m_cand : m
//     p_ij   = exp2(fma(F_ij, ct, nk)) (<= 2^8, fits E4M3), ct = cl * KS_block
//     l      = corr * l + sum_j p_ij (fp32 p);  O = need ? O * corr : O;  O += e4m3(p) V8;  corr = exp2((m - m_new) cl)
//   out    = (O * ((1/448) / l)) * VS
// Scores.  Head dims up to 128 seed the QK accumulators with the bit pattern of c = fp32(1 / (2 pi)) = 0x3E22F983,
// an inline constant of the MFMA (no registers hold the seed): since -2,292,099 <= S <= 6,096,509 there, the int32
// result stays inside c's binade [1/8, 1/4] (ulp 2^-26; its ends read right), so read as fp32 it is
// F = c + S * 2^-26 and needs no conversion; nk = -(cl * m_new) - fp32(c * ct), so F * ct + nk equals
// S * ct - cl * m_new up to the rounding of nk.  Those kernels keep cl scaled by 2^26 and m by 2^-26 (powers of
// two: every product and difference of the math above is the same bits, scaled).  Head dim 256 reaches |S| = 4,129,024, outside that binade, so its
// accumulators start at 0 and F = fp32(S) (v_cvt_f32_i32), nk = -(cl * m_new): the reference's arithmetic.  The
// rounding of fp32(c * ct) grows with the input scale; a wave whose scales are large enough for it to matter reads
// F - c = S * 2^-26 (exact) with nk = -(cl * m_new) instead (the `wide` test, once per work unit).
// Passes.  Once every row of a wave has a max, a tile first runs without the block maxima: p with the current m,
// kept when every lane's sum of 16 probabilities of each block stays below 2^7.5 (then no row's max can move), else
// redone exactly (the maxima, the lazy-rescale decisions above, and a second pass when block 1 rescales).
// Split tiles (the short last round of a launch): contiguous key ranges in parallel, merged by attn_merge_kernel; a
// range after the block's first visited key tile starts from the max the one walk over every key has after that
// tile (not from -inf), so it forms the walk's own probabilities wherever that max stays put.
//
// gfx950 mapping.  A workgroup owns 128 query rows (4 waves x 32) of one (batch, head) and walks the KV sequence
// in 64-key tiles staged in LDS by direct global -> LDS loads (three buffers at head dims up to 128, the loads of the
// next two tiles in flight while one is computed; two at 256 and in the mask variant).  Per wave and tile:
//   * S^T = K Q^T with v_mfma_i32_32x32x32_i8: A = 32 keys x 32 dims of K (LDS), B = 32 dims x 32 queries of Q
//     (registers for the whole kernel).  The 32x32 accumulator gives lane l the query l % 32 and 16 keys
//     8(v/4) + 4(l/32) + v%4 of the block (v = accumulator register), so row statistics need one exchange with lane
//     l ^ 32 (v_permlane32_swap) and no other cross-lane traffic.
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

// chunk swizzle for LDS rows of `row_bytes` (64, 128 or 256)
template <int ROW_BYTES> __device__ __forceinline__ int swz(int row, int chunk) {
  if (ROW_BYTES == 256) return chunk ^ (row & 15);
  if (ROW_BYTES == 128) return chunk ^ ((row >> 1) & 7);
  return chunk ^ ((row >> 2) & 3);
}

// workgroups per CU the launch bounds ask for: d256 tiles take 64 KiB of LDS and twice the accumulators
template <int D> constexpr int attn_occupancy() { return D == 256 ? 2 : 3; }

// Direct global -> LDS copy of 16 bytes per lane: the data lands at LDS address (M0 base) + 16 * lane, so a wave
// writes one contiguous KiB; `lds` must be wave-uniform.
__device__ __forceinline__ void copy16_to_lds(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// 32-bit load through the global address space (a generic pointer would give a flat load, which also counts on the
// LDS counter, so every LDS wait of the tile would wait for it)
__device__ __forceinline__ uint32_t load_global_u32(const uint8_t* p) {
  return *(const __attribute__((address_space(1))) uint32_t*)(p);
}

// 16 bytes through the global address space
__device__ __forceinline__ v4i load_global_v4i(const uint8_t* p) {
  return *(const __attribute__((address_space(1))) v4i*)(p);
}

// an additive mask element (the input dtype's 16 bits in the low half) as fp32
template <int DT> __device__ __forceinline__ float mask_half_to_f32(uint32_t h) {
  if constexpr (DT == DT_BF16)
    return __uint_as_float(h << 16);
  else
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// First QK MFMA of a key block: C = the seed as the instruction's inline constant (the bits of fp32(1 / (2 pi)),
// or 0 for the unseeded head dim 256).  The compiler folds a splat of it into the MFMA only where the splat has a
// single use; the second block's MFMA would make it a 16-register value live through the whole tile loop, so that
// one is written out.  Its result is read only as the exactly overlapping C operand of the block's next MFMA, which
// needs no wait states.
template <bool SEEDED> __device__ __forceinline__ v16i mfma_i8_seeded(v4i a, v4i b) {
  v16i d;
  if constexpr (SEEDED)
    asm("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0.15915494" : "=&v"(d) : "v"(a), "v"(b));
  else
    asm("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}

// Whether the QK accumulators of a kernel covering `da` channels start at the seed c = fp32(1 / (2 pi)).  The int32
// sum read as fp32 is c + S * 2^-26 exactly while it stays inside c's binade [1/8, 1/4] (the ends read right), i.e. for
// -2,292,099 <= S <= 6,096,509 (c = 10,680,707 * 2^-26).  |S| <= 127^2 * da: 1,032,256 (64), 1,548,384 (96, zero
// padded), 2,064,512 (128) fit; head dim 256 reaches 4,129,024 and converts S with v_cvt_f32_i32 instead.
__host__ __device__ constexpr bool attn_seeded(int da) { return 127 * 127 * da < 2292099; }

constexpr int ATT_MAX_CHUNKS = 16;

// Workspace of a split launch (units = split tiles x chunks): each chunk's O normalised by its own l, as fp16
// [units][128 rows][D] (|O / l| <= 448, the E4M3 range of V8), then (m, l) as float2 [units][128 rows].
__host__ __device__ constexpr int64_t ws_ml_offset(int64_t units, int D) { return units * ATT_BM * D * 2; }
__host__ __device__ constexpr int64_t ws_bytes(int64_t units, int D) { return units * ATT_BM * (2 * D + 8); }

// Packed variable-length sequences (VARLEN): block i runs tile tiles[i] = (sequence, head, query tile) or exits when
// its sequence is -1.  Q8 / QS rows are [H][TQ] (TQ = the `Sq` argument), K8 / KS / V8T the padded packed layout
// of the quantizer (kv head stride / V8T channel stride `Skp` = TKP, sequence b from row kp[b]), VS [batch][Hkv][D],
// output rows cu_q[b] + i with strides (oss, osh).
struct VarlenTiles {
  const int4* tiles;  // (sequence, head, query tile, 0) per block
  const int* cu_q;    // [batch + 1]
  const int* cu_k;    // [batch + 1]
  const int* kp;      // [batch + 1] padded key offsets
};


// HD is the head dim; D = layout_dim(HD) the channel count of the Q8 / K8 / V8T layouts (128 for head_dim 96, whose
// rows are zero-padded) and DA = HD the channels the MFMAs cover: the zero channels of head_dim 96 add nothing to S
// and give output channels that are not written, so its tiles run 3 of the 4 QK and PV MFMA blocks of the 128-channel
// layout.  `dout` output channels are written.  c0 = log2(e) / sqrt(head_dim).
// MASK: a boolean mask (MaskTabs) instead of the causal / padding bound; the causal flag is folded into its bits.
template <int HD, bool CAUSAL, int OUT_DT, bool VARLEN, bool MASK = false>
__global__ __launch_bounds__(ATT_THREADS, attn_occupancy<layout_dim(HD)>()) void attn_kernel(
    const int8_t* __restrict__ q8, const float* __restrict__ qs, const int8_t* __restrict__ k8,
    const float* __restrict__ ks, const uint8_t* __restrict__ v8t, const float* __restrict__ vs,
    uint16_t* __restrict__ out, int64_t osb, int64_t oss, int64_t osh, float* __restrict__ lse, int H, int Hkv,
    int Sq_arg, int Skv_arg, int Skp, int q_tiles, int total, int n_full, int chunks, float* __restrict__ part,
    float c0, int dout, VarlenTiles vt, MaskTabs mt, const uint32_t* __restrict__ mbits_tab,
    const int* __restrict__ mcls_tab, const int2* __restrict__ mrange_tab, const uint16_t* __restrict__ mbias_tab) {
  static_assert(!(MASK && (CAUSAL || VARLEN)), "the mask variant folds causality into its bits and is dense only");
  constexpr int D = layout_dim(HD);
  constexpr int DA = HD;
  constexpr int BN = ATT_BN;
  constexpr int KTILE = BN * D;      // bytes of the K tile  ([64 keys][D], 16-byte chunks XOR-swizzled per row)
  constexpr int VTILE = D * BN;      // bytes of the V tile  ([D channels][64 keys])
  constexpr int TILE = KTILE + VTILE;
  constexpr int NQK = DA / 32;       // i8 MFMAs (K = 32 dims) per 32-key block
  constexpr int NPV = DA / 32;       // fp8 MFMAs (M = 32 channels) per tile
  constexpr int KCH = D / 16;        // 16-byte chunks per K row
  constexpr int KLOADS = KTILE / 1024 / 4;  // 1 KiB direct loads per wave per tile (4 waves)
  constexpr int VLOADS = VTILE / 1024 / 4;
  // Seeded scores (F = c + S * 2^-26, c = fp32(1 / (2 pi))): cl is kept scaled by 2^26 and m by 2^-26.  Unseeded
  // (head dim 256): F = fp32(S) from v_cvt_f32_i32, no scaling, which is the reference's fp32(S) exactly.
  constexpr bool SEEDED = attn_seeded(DA);
  constexpr uint32_t SEED_BITS = SEEDED ? 0x3E22F983u : 0u;
  constexpr float SEED_F = __builtin_bit_cast(float, SEED_BITS);
  constexpr float SSCALE = SEEDED ? 67108864.0f : 1.0f;  // 2^26
  // Passes of a tile body: speculative (the offsets of the current m, no block maxima), exact (the block maxima and
  // the reference's rescale decisions), and the redo of block 1 after a block-1 rescale.  Head dim 256 (which would
  // spill with the speculative code) and the additive-mask body (MODE 3, whose row maxima are taken over the biased
  // logits it forms in the same loop) have no speculative pass.
  constexpr int PASS_NONE = 0, PASS_SPEC = 1, PASS_EXACT = 2, PASS_REDO = 3;
  constexpr bool SPEC_OK = HD <= 128;
  constexpr float SPEC_SUM = 181.0f;  // below 2^7.5: a margin of 2^0.5 under the threshold for fp32 rounding
  constexpr float CT_WIDE = 262144.0f;  // 2^18: the largest ct (scaled by 2^26) read through the seeded form
  // K / V tile buffers: three where they fit (the unmasked loops prefetch two tiles ahead, which hides the direct
  // loads' latency behind two tiles of arithmetic), two for head dim 256 (3 x 32 KiB per workgroup would leave room
  // for one workgroup per CU) and for the mask variant (whose loops prefetch one tile ahead)
  constexpr int NBUF = (!MASK && D <= 128) ? 3 : 2;
  constexpr int LPT = KLOADS + VLOADS;  // direct loads per wave and tile
  __shared__ __attribute__((aligned(16))) uint8_t smem[NBUF][TILE];

  // ---- work decode.  Dense: blocks [0, n_full) own whole query tiles (XCD-grouped); each later block owns one of
  // the `chunks` key ranges of a split tile.  VARLEN: the tile table. ----
  const bool split = !VARLEN && (int)blockIdx.x >= n_full;
  int b, h, qt, unit = 0, Sq = Sq_arg, Skv = Skv_arg;
  int64_t qrow0;       // Q8 / QS row of query 0 of this (sequence, head)
  int khead, kofs;     // K8 / KS / V8T head index and the sequence's first key row inside it
  uint16_t* obase;
  if (VARLEN) {
    const int4 e = vt.tiles[blockIdx.x];
    if (e.x < 0) return;
    b = e.x;
    h = e.y;
    qt = e.z;
    const int qb = vt.cu_q[b];
    Sq = vt.cu_q[b + 1] - qb;
    Skv = vt.cu_k[b + 1] - vt.cu_k[b];
    qrow0 = (int64_t)h * Sq_arg + qb;
    khead = h / (H / Hkv);
    kofs = vt.kp[b];
    obase = out + (int64_t)qb * oss;
  } else {
    int bh;
    if (CAUSAL) {
      causal_tile(blockIdx.x, total / q_tiles, q_tiles, bh, qt);  // causal launches are never split
    } else {
      int logical;
      if (!split) {
        logical = xcd_remap(blockIdx.x, n_full);
      } else {
        unit = blockIdx.x - n_full;
        logical = n_full + unit / chunks;
      }
      bh = logical / q_tiles;
      qt = logical % q_tiles;
    }
    b = bh / H;
    h = bh % H;
    qrow0 = (int64_t)bh * Sq;
    khead = b * Hkv + h / (H / Hkv);
    kofs = 0;
    obase = out + b * osb;
  }
  const int hkv = h / (H / Hkv);
  const int bhk = b * Hkv + hkv;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, hf = lane >> 5;
  const int q0 = qt * ATT_BM + wave * 32;
  const int qrow = q0 + ln;
  const bool qvalid = qrow < Sq;
  const int qr = qvalid ? qrow : Sq - 1;
  const int off = Skv - Sq;  // bottom-right causal offset

  // ---- Q operand (B of the QK MFMA): lane (query ln, half hf) holds dims [32i + 16hf, +16) ----
  v4i qa[NQK];
  {
    const int8_t* qp = q8 + (qrow0 + qr) * D + 16 * hf;
#pragma unroll
    for (int i = 0; i < NQK; ++i) qa[i] = *reinterpret_cast<const v4i*>(qp + 32 * i);
  }
  const float qsv = qs[qrow0 + qr];
  // The K scales of the keys [0, Skv), whose maximum decides `wide` below: the first 256 blocks loaded four per lane
  // beside the Q operand and its scale (one wait for all), the rest (long key ranges only) eight per lane at a time
  const float* ksq = ks + ((int64_t)khead * Skp + kofs) / SAGE_KV_BLOCK;
  const int nkb = (Skv + SAGE_KV_BLOCK - 1) / SAGE_KV_BLOCK;
  float kq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // a packed sequence without keys (nkb = 0) reads no scale: its tile loop is empty and `wide` stays false
  if (SEEDED && nkb > 0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) kq[u] = ksq[min(64 * u + lane, nkb - 1)];
  }
  // cl of the math scaled by SSCALE, m in units of S * ks / SSCALE (the seeded accumulators below hold S * 2^-26)
  const float cl = (c0 * qsv) * SSCALE;
  const float rcl = 1.0f / cl;  // the bias tiles keep m in S * ks * 2^-26 units
  // Large scales.  The seeded exponent argument fma(F, ct, -(cl * m) - fp32(c * ct)) carries the rounding of c * ct,
  // up to ~1.5 ct * 2^-26 log2 units, which grows with the input scale (~2^-9 at ct = 2^18; the benchmark inputs
  // stay below 2.5e4).  A wave whose largest K scale of the keys [0, Skv) exceeds fp32(CT_WIDE / its largest cl)
  // reads its scores exactly instead, F - c = S * 2^-26 (Sterbenz), with the offset -(cl * m): the reference's
  // fma(S, cl * ks, -cl * m).  Decided once per work unit; both maxima are of positive floats, so their bit
  // patterns order like unsigned ints.
  bool wide = false;
  if (SEEDED) {
    float km = fmaxf(fmaxf(kq[0], kq[1]), fmaxf(kq[2], kq[3]));
    for (int j0 = 256; j0 < nkb; j0 += 512) {
      float kx[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kx[u] = ksq[min(j0 + 64 * u + lane, nkb - 1)];
#pragma unroll
      for (int u = 0; u < 8; ++u) km = fmaxf(km, kx[u]);
    }
    const float cmx = wave_max_pos(cl), kmx = wave_max_pos(km);
    wide = kmx > CT_WIDE / cmx;
  }

  // ---- KV range ----
  int kv_end = Skv;
  if (CAUSAL) kv_end = max(0, min(Skv, qt * ATT_BM + ATT_BM + off));  // 0: no row of the tile sees a key
  const int ntiles = (kv_end + BN - 1) / BN;
  int t_lo = 0, t_hi = ntiles;
  if (split) {
    const int ch = unit % chunks;
    t_lo = ch * ntiles / chunks;
    t_hi = (ch + 1) * ntiles / chunks;
  }

  // ---- mask: this lane's bit row and this wave's class row; the workgroup runs only the tiles from the first to the
  // last that any of its rows sees (mask_range_block; the tiles outside hold no visible key, so skipping them is
  // exactly the online softmax over them) ----
  const uint8_t* mbase = nullptr;  // this (batch, head)'s mask words; the lane's row at byte offset moff
  uint32_t moff = 0;                 // (a (batch, head) slice of the bits is below 2 GiB, checked on the host)
  const uint8_t* bbase = nullptr;  // the same for the bias values of an additive mask (64 bytes per word)
  uint32_t boff = 0;
  const int* mcls = nullptr;
  int mseed_tile = -1;  // MASK: the tile whose full pass seeds a split range's running max (-1: none)
  if (MASK) {
    const int64_t wslice = (int64_t)b * mt.bsb + (int64_t)h * mt.bsh;
    mbase = reinterpret_cast<const uint8_t*>(mbits_tab + wslice);
    moff = (uint32_t)(((int64_t)qr * mt.bsq + hf) * 4);
    bbase = reinterpret_cast<const uint8_t*>(mbias_tab + wslice * 32);
    boff = (uint32_t)(((int64_t)qr * mt.bsq + hf) * 64);
    mcls = mcls_tab + (int64_t)b * mt.csb + (int64_t)h * mt.csh + (int64_t)min(q0 >> 5, mt.groups - 1) * mt.csg;
    const int2 r = mrange_tab[(int64_t)b * mt.rsb + (int64_t)h * mt.rsh + min(qt, mt.rblocks - 1)];
    // a split range after the block's first visited tile starts from the walk's max after that tile (below)
    if (split && t_lo > r.x && r.x < r.y) mseed_tile = r.x;
    t_lo = max(t_lo, r.x);
    t_hi = min(t_hi, r.y);
  }

  const int8_t* kbase = k8 + ((int64_t)khead * Skp + kofs) * D;
  const uint8_t* vbase = v8t + (int64_t)khead * D * Skp + kofs;
  const float* ksb = ks + ((int64_t)khead * Skp + kofs) / SAGE_KV_BLOCK;
  // Source of each lane's direct loads.  Load j of wave w fills LDS chunk L = (w * LOADS + j) * 64 + lane of the
  // region, which must receive the tile chunk that the swizzled layout stores there.
  uint32_t koff[KLOADS];
  uint32_t voff[VLOADS];  // D * Skp < 2^31 (checked on the host)
#pragma unroll
  for (int j = 0; j < KLOADS; ++j) {
    const int L = (wave * KLOADS + j) * 64 + lane;
    const int row = L / KCH;
    koff[j] = (uint32_t)(row * D + swz<D>(row, L % KCH) * 16);  // swz is an involution: stored chunk c' holds chunk c' ^ s
  }
#pragma unroll
  for (int j = 0; j < VLOADS; ++j) {
    const int L = (wave * VLOADS + j) * 64 + lane;
    const int d = L >> 2;
    voff[j] = (uint32_t)(d * Skp + swz<BN>(d, L & 3) * 16);
  }
#define SAGE_ISSUE_TILE(T, BUF)                                                                            \
  do {                                                                                                     \
    const int tt_ = (T);                                                                                   \
    uint8_t* dst_ = smem[BUF];                                                                             \
    /* uniform bases pinned to SGPRs and offsets widened here (not hoisted as 64-bit values): each load is    \
       then the SGPR-pair base + 32-bit lane offset form, with no 64-bit address registers */                \
    const int8_t* kb_ = kbase + (int64_t)tt_ * KTILE;                                                      \
    const uint8_t* vb_ = vbase + tt_ * BN;                                                                 \
    asm volatile("" : "+s"(kb_), "+s"(vb_));                                                               \
    _Pragma("unroll") for (int j_ = 0; j_ < KLOADS; ++j_) {                                                \
      asm volatile("" : "+v"(koff[j_]));                                                                 \
      copy16_to_lds(kb_ + koff[j_], dst_ + (wave * KLOADS + j_) * 1024);                                    \
    }                                                                                                      \
    _Pragma("unroll") for (int j_ = 0; j_ < VLOADS; ++j_) {                                                \
      asm volatile("" : "+v"(voff[j_]));                                                                 \
      copy16_to_lds(vb_ + voff[j_], dst_ + KTILE + (wave * VLOADS + j_) * 1024);                            \
    }                                                                                                      \
  } while (0)

  // Lane-constant LDS offsets of the MFMA operands.  For rows 32 kb + ln the K swizzle does not depend on kb, and
  // for channel rows 32 j + ln the V swizzle does not depend on j, so one offset per step serves every block.
  int ko[NQK];
#pragma unroll
  for (int i = 0; i < NQK; ++i) ko[i] = ln * D + swz<D>(ln, 2 * i + hf) * 16;
  const int vo0 = ln * BN + swz<BN>(ln, 2 * hf) * 16;
  const int vo1 = ln * BN + swz<BN>(ln, 2 * hf + 1) * 16;

  v16f o[NPV];
#pragma unroll
  for (int i = 0; i < NPV; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[i][v] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  float negm = 0.0f;  // -(cl * m_ref), m_ref = m or 0 while m = -inf: the exponent offset while m stays
  bool fastok = false;  // every lane of the wave has a finite m: its tiles start with a speculative pass
  v8i pb = {};  // E4M3 probabilities (B operand of the PV MFMA); each cvt rewrites one half, so no clearing
  v4i bw_none[4] = {};  // the bias argument of the tile bodies without an additive mask (never read)

  // One tile: S^T = K Q^T (int8 MFMA), online softmax with the reference's lazy rescale, O^T += V^T P^T (fp8 MFMA).
  // The wave raises its issue priority over each run of MFMAs, so that a wave with MFMAs ready feeds the matrix
  // core ahead of the softmax arithmetic of the SIMD's other waves.
  // MODE 0: every key visible; 1: keys beyond the causal / padding bound masked; 2: keys whose bit of MW is clear
  // masked (MW = the lane's mask word of the tile); 3: the additive mask values BW (the lane's 32 16-bit values,
  // input dtype, -inf = masked) added in log2 units, with the row max taken over the biased logits.
  // The rescale decision is taken once per 32-key block, as the reference's 32-key tiles take it
  // (kernel_build/make_sage_r2.py:180-190): block 0 against m, block 1 against the max m1 that block 0 left.  Once
  // every lane of the wave has a finite m, a tile starts with a speculative pass (PASS_SPEC) that takes no block
  // maxima: it forms the probabilities with the current m and stands when every lane's sums are small enough that
  // no row's max can have moved (almost every tile); otherwise it adds nothing and the tile runs an exact pass.  In
  // an exact pass (PASS_EXACT) a wave-uniform test first asks whether any lane's larger block max moves its max at
  // all; if none does, m, the exponent offset negm and l's scale stay as they are (no per-block work).  Otherwise the
  // per-block decisions run.  When no lane moves its max at block 1, one K = 64 PV MFMA per channel block adds both
  // blocks (the reference's two PV steps up to the fp32 summation order).  When some lane does (rare: a row's max
  // rising by 2^8 inside a tile), the wave runs the tile body again before the tile's barrier: the exact pass adds
  // block 0 alone (block 1's exponent offset is -inf, so its probabilities, sum and E4M3 bytes are 0, and m = m1),
  // the redo pass (PASS_REDO) masks block 0 and adds block 1, whose rescale then comes before its MFMA.  No MFMA
  // sits in a branch: around one the compiler
  // loses the accumulators' coalescing and spills the whole loop; the O rescale sits in its own branch after the
  // exponentials for the same reason.
#define SAGE_TILE(T, MODE, MW, BW, KIND, WIDE)                                                             \
  do {                                                                                                     \
    const int t_ = (T);                                                                                    \
    const uint8_t* kt_ = smem[t_ % NBUF];                                                                  \
    const uint8_t* vt_ = smem[t_ % NBUF] + KTILE;                                                          \
    v16i s_[2];                                                                                            \
    __builtin_amdgcn_s_setprio(1);                                                                         \
    _Pragma("unroll") for (int i_ = 0; i_ < NQK; ++i_) {                                                   \
      const v4i k0_ = *reinterpret_cast<const v4i*>(kt_ + ko[i_]);                                         \
      const v4i k1_ = *reinterpret_cast<const v4i*>(kt_ + ko[i_] + 32 * D);                                \
      s_[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(k0_, qa[i_], i_ == 0 ? seed16 : s_[0], 0, 0, 0);       \
      s_[1] = i_ == 0 ? mfma_i8_seeded<SEEDED>(k1_, qa[i_])                                                \
                      : __builtin_amdgcn_mfma_i32_32x32x32_i8(k1_, qa[i_], s_[1], 0, 0, 0);                \
    }                                                                                                      \
    __builtin_amdgcn_s_setprio(0);                                                                         \
    float sf_[2][16];                                                                                      \
    _Pragma("unroll") for (int kb_ = 0; kb_ < 2; ++kb_)                                                    \
      _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_)                                                    \
        sf_[kb_][v_] = SEEDED ? __int_as_float(s_[kb_][v_]) : (float)s_[kb_][v_];                          \
    if ((MODE) == 1) {                                                                                     \
      /* element (kb, v) holds key t * 64 + 4 hf + c with the constant c = 32 kb + 8 (v / 4) + v % 4; it is    \
         visible iff key <= min(Skv - 1, qr + off), i.e. c <= lim (one 32-bit bound per tile and lane) */   \
      const int lim_ = (CAUSAL ? min(Skv - 1, qr + off) : Skv - 1) - (t_ * BN + 4 * hf);                   \
      _Pragma("unroll") for (int kb_ = 0; kb_ < 2; ++kb_)                                                  \
        _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                                \
          if (32 * kb_ + 8 * (v_ >> 2) + (v_ & 3) > lim_) sf_[kb_][v_] = -INFINITY;                        \
        }                                                                                                  \
    }                                                                                                      \
    if ((MODE) == 2) {                                                                                     \
      /* keep = all ones where bit 16 kb + v of the word is set: one extract and one bit select per score */ \
      _Pragma("unroll") for (int kb_ = 0; kb_ < 2; ++kb_)                                                  \
        _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                                \
          const int keep_ = __builtin_amdgcn_sbfe((int)(MW), 16 * kb_ + v_, 1);                            \
          sf_[kb_][v_] = __int_as_float((__float_as_int(sf_[kb_][v_]) & keep_) | (int)(0xFF800000u & ~(uint32_t)keep_)); \
        }                                                                                                  \
    }                                                                                                      \
    if ((KIND) == PASS_REDO) {                                                                             \
      _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) sf_[0][v_] = -INFINITY;                            \
    }                                                                                                      \
    const float ks0_ = ksb[2 * t_], ks1_ = ksb[2 * t_ + 1];                                                \
    const float ct0_ = cl * ks0_, ct1_ = cl * ks1_;                                                        \
    /* the blocks' exponent offsets (MODE 3: added to t) while m stays: -(cl * m_ref) - fp32(c * ct) (seeded), \
       -(cl * m_ref) (unseeded, and MODE 3 whose t holds the seed term) */                                 \
    float nk0_ = ((MODE) != 3 && SEEDED) ? negm - SEED_F * ct0_ : negm;                                    \
    float nk1_ = ((MODE) != 3 && SEEDED) ? negm - SEED_F * ct1_ : negm;                                    \
    float corr_ = 1.0f;     /* the rescale before this pass's MFMA */                                      \
    bool slow_ = false;     /* some lane moves its max at block 1 in a first pass: block 1 waits for pass 1 */ \
    bool resc_ = false;     /* some lane rescales O before this pass's MFMA */                             \
    const bool spec_ = SPEC_OK && (MODE) != 3 && (KIND) == PASS_SPEC;                                      \
    if (!spec_) {                                                                                          \
      /* the two 32-key blocks' row maxima, one per lane half (block hf's, for row ln): MODE 3 in log2 units of the \
         biased logits t (kept in sf_), else in m's units, fp32(max S * ks) (scaled by 2^-26 when seeded: mx - c is \
         exact).  One lane exchange gives block 0's max in lanes 0-31 and block 1's in lanes 32-63. */     \
      float bmh_;                                                                                          \
      if ((MODE) == 3) {                                                                                   \
        /* t = fma(F, ct, fma(b, log2e, -fp32(c * ct))) (b = -inf for a masked key gives -inf); the lazy   \
           rescale compares a block's max of t with m * cl and keeps m in S * ks units (m_new = m_cand / cl) */ \
        float ns0_ = SEEDED ? -(SEED_F * ct0_) : -0.0f, ns1_ = SEEDED ? -(SEED_F * ct1_) : -0.0f;          \
        if (WIDE) {  /* exact scores, no seed term */                                                      \
          ns0_ = ns1_ = -0.0f;                                                                             \
          _Pragma("unroll") for (int kb_ = 0; kb_ < 2; ++kb_)                                              \
            _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) sf_[kb_][v_] -= SEED_F;                      \
        }                                                                                                  \
        float tm0_ = -INFINITY, tm1_ = -INFINITY;                                                          \
        _Pragma("unroll") for (int kb_ = 0; kb_ < 2; ++kb_)                                                \
          _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                              \
            const uint32_t bw_ = (BW)[(16 * kb_ + v_) >> 3][((16 * kb_ + v_) >> 1) & 3];                   \
            const float b_ = mask_half_to_f32<OUT_DT>((v_ & 1) ? (bw_ >> 16) : (bw_ & 0xFFFFu));           \
            const float in_ = __builtin_fmaf(b_, 1.44269504088896341f, kb_ ? ns1_ : ns0_);                 \
            sf_[kb_][v_] = __builtin_fmaf(sf_[kb_][v_], kb_ ? ct1_ : ct0_, in_);                           \
            if (kb_) tm1_ = fmaxf(tm1_, sf_[kb_][v_]);                                                     \
            else tm0_ = fmaxf(tm0_, sf_[kb_][v_]);                                                         \
          }                                                                                                \
        bmh_ = halves_max_f32(tm0_, tm1_);                                                                 \
      } else {                                                                                             \
        float mxh_;                                                                                        \
        if (SEEDED) {                                                                                      \
          /* block maxima on the bit patterns: the scores are positive floats (c + S * 2^-26) or -inf, whose \
             int32 patterns order like the floats, and an integer max needs no NaN canonicalisation */     \
          int mi0_ = __float_as_int(sf_[0][0]), mi1_ = __float_as_int(sf_[1][0]);                          \
          _Pragma("unroll") for (int v_ = 1; v_ < 16; ++v_) {                                              \
            mi0_ = max(mi0_, __float_as_int(sf_[0][v_]));                                                  \
            mi1_ = max(mi1_, __float_as_int(sf_[1][v_]));                                                  \
          }                                                                                                \
          mxh_ = __int_as_float(halves_max_i32(mi0_, mi1_));                                               \
        } else {                                                                                           \
          float mx0_ = sf_[0][0], mx1_ = sf_[1][0];                                                        \
          _Pragma("unroll") for (int v_ = 1; v_ < 16; ++v_) {                                              \
            mx0_ = fmaxf(mx0_, sf_[0][v_]);                                                                \
            mx1_ = fmaxf(mx1_, sf_[1][v_]);                                                                \
          }                                                                                                \
          mxh_ = halves_max_f32(mx0_, mx1_);                                                               \
        }                                                                                                  \
        const float ksh_ = hf ? ks1_ : ks0_;                                                               \
        bmh_ = SEEDED ? (mxh_ - SEED_F) * ksh_ : mxh_ * ksh_;                                              \
      }                                                                                                    \
      /* Does some lane of the wave move its max at either block?  The ballot over both lane halves covers both \
         blocks of every row (an -inf max against m = -inf gives NaN, false, as the per-block test does).  Then \
         m stays, and so does the exponent offset negm = -(cl * m_ref). */                                 \
      const bool any_ = __ballot((MODE) == 3 ? (bmh_ - m * cl) > 8.0f : (bmh_ - m) * cl > 8.0f) != 0;      \
      if (any_) {                                                                                          \
        /* the reference's decisions, block 0 against m, block 1 against the max m1 block 0 left */        \
        float bm0_, bm1_;                                                                                  \
        halves_split_f32(bmh_, bm0_, bm1_);                                                                \
        bool need0_, need1_;                                                                               \
        float m1_, m2_;                                                                                    \
        if ((MODE) == 3) {                                                                                 \
          const float mc0_ = m * cl;                                                                       \
          const float mcand0_ = fmaxf(mc0_, bm0_);                                                         \
          need0_ = (mcand0_ - mc0_) > 8.0f;                                                                \
          m1_ = need0_ ? mcand0_ * rcl : m;                                                                \
          const float mc1_ = m1_ * cl;                                                                     \
          const float mcand1_ = fmaxf(mc1_, bm1_);                                                         \
          need1_ = (mcand1_ - mc1_) > 8.0f;                                                                \
          m2_ = need1_ ? mcand1_ * rcl : m1_;                                                              \
        } else {                                                                                           \
          const float mcand0_ = fmaxf(m, bm0_);                                                            \
          need0_ = (mcand0_ - m) * cl > 8.0f;                                                              \
          m1_ = need0_ ? mcand0_ : m;                                                                      \
          const float mcand1_ = fmaxf(m1_, bm1_);                                                          \
          need1_ = (mcand1_ - m1_) * cl > 8.0f;                                                            \
          m2_ = need1_ ? mcand1_ : m1_;                                                                    \
        }                                                                                                  \
        /* a row that has seen no key yet (possible only in masked tiles) keeps m = -inf and p = 0: offsets \
           from 0 instead of -inf keep corr and the exponents free of NaN */                               \
        const float mref1_ = m1_ == -INFINITY ? 0.0f : m1_;                                                \
        const float mref2_ = m2_ == -INFINITY ? 0.0f : m2_;                                                \
        slow_ = (KIND) != PASS_REDO && __ballot(need1_) != 0;                                              \
        /* nk = -(cl * m_new) - fp32(c * ct) (seeded), -(cl * m_new) (unseeded, and MODE 3 whose t holds the \
           seed term); in a slow first pass block 1's offset is -inf, so its p, sum and E4M3 bytes are 0 */ \
        const float neg1_ = 0.0f - cl * mref1_, neg2_ = 0.0f - cl * mref2_;                                \
        nk0_ = ((MODE) != 3 && SEEDED) ? neg1_ - SEED_F * ct0_ : neg1_;                                    \
        nk1_ = slow_ ? -INFINITY : (((MODE) != 3 && SEEDED) ? neg2_ - SEED_F * ct1_ : neg2_);              \
        /* exp2(carg0 + carg1) with carg1 counted unless slow; one of the two is 0 wherever a row has seen a \
           key (a non-slow first pass has no block-1 rescale, a redo pass's masked block 0 none at block 0), so \
           this is the reference's corr0 or corr1; 1 in a lane whose max does not move */                  \
        const float carg0_ = (m - mref1_) * cl, carg1_ = (m1_ - mref2_) * cl;                              \
        resc_ = __ballot(need0_ || (!slow_ && need1_)) != 0;                                               \
        if (resc_) corr_ = __builtin_amdgcn_exp2f(carg0_ + (slow_ ? 0.0f : carg1_));                       \
        m = slow_ ? m1_ : m2_;                                                                             \
        negm = 0.0f - cl * (m == -INFINITY ? 0.0f : m);                                                    \
      }                                                                                                    \
      if (SPEC_OK) fastok = __ballot(m == -INFINITY) == 0;                                                 \
    }                                                                                                      \
    /* p = exp2(arg); each block's fp32 sum starts from its first p (0 + p is p).  Up to head dim 128 and   \
       without a mask all 32 exponent arguments are formed before the first exponential (SAGE_PHASE_FENCE):  \
       interleaved, each v_exp_f32 waits on the FMA just before it, which three waves per SIMD do not hide.   \
       The mask variant (three tile bodies) and head dim 256 hold more registers and would spill with it. */ \
    /* a wide wave reads F - c after the block maxima (which order the seeded patterns as ints) and drops the \
       seed term: the offsets are then -(cl * m) after this pass's update, -inf for a slow pass's block 1 */ \
    if ((MODE) != 3 && (WIDE)) {                                                                           \
      nk0_ = negm;                                                                                         \
      nk1_ = slow_ ? -INFINITY : negm;                                                                     \
      _Pragma("unroll") for (int kb_ = 0; kb_ < 2; ++kb_)                                                  \
        _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) sf_[kb_][v_] -= SEED_F;                          \
    }                                                                                                      \
    float psum0_, psum1_;                                                                                  \
    _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                                    \
      sf_[0][v_] = (MODE) == 3 ? sf_[0][v_] + nk0_ : __builtin_fmaf(sf_[0][v_], ct0_, nk0_);               \
      sf_[1][v_] = (MODE) == 3 ? sf_[1][v_] + nk1_ : __builtin_fmaf(sf_[1][v_], ct1_, nk1_);               \
    }                                                                                                      \
    if constexpr (!MASK && HD <= 128) SAGE_PHASE_FENCE(sf_);                                               \
    _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                                    \
      sf_[0][v_] = __builtin_amdgcn_exp2f(sf_[0][v_]);                                                     \
      sf_[1][v_] = __builtin_amdgcn_exp2f(sf_[1][v_]);                                                     \
    }                                                                                                      \
    _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                                    \
      psum0_ = v_ == 0 ? sf_[0][0] : psum0_ + sf_[0][v_];                                                  \
      psum1_ = v_ == 0 ? sf_[1][0] : psum1_ + sf_[1][v_];                                                  \
    }                                                                                                      \
    if (resc_) {                                                                                           \
      _Pragma("unroll") for (int i_ = 0; i_ < NPV; ++i_)                                                   \
        _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) o[i_][v_] *= corr_;                              \
    }                                                                                                      \
    /* a speculative pass stands only if every lane's sum of its 16 probabilities of each block is below 2^7.5: \
       then every p is, so no row's block max exceeds m by the rescale threshold 2^8 and the reference keeps m. \
       Otherwise the pass adds nothing (l stays, the E4M3 bytes are zeroed so the MFMA adds +-0 to O, which \
       never holds -0) and the tile runs as an exact pass. */                                              \
    /* one ballot per compare: each is the compare's lane mask, where a ballot of their OR costs a select */ \
    const uint64_t big_ = __builtin_amdgcn_ballot_w64(!(psum0_ < SPEC_SUM)) |                              \
                          __builtin_amdgcn_ballot_w64(!(psum1_ < SPEC_SUM));                               \
    const bool sfail_ = spec_ && big_ != 0;                                                                \
    if (sfail_) {                                                                                          \
      _Pragma("unroll") for (int w_ = 0; w_ < 8; ++w_) pb[w_] = 0;                                         \
    } else {                                                                                               \
      l = (corr_ * l + psum0_) + psum1_;                                                                   \
      _Pragma("unroll") for (int w_ = 0; w_ < 8; ++w_) {                                                   \
        const int kb_ = w_ >> 2, v0_ = 4 * (w_ & 3);                                                       \
        pb[w_] = __builtin_amdgcn_cvt_pk_fp8_f32(sf_[kb_][v0_], sf_[kb_][v0_ + 1], pb[w_], false);         \
        pb[w_] = __builtin_amdgcn_cvt_pk_fp8_f32(sf_[kb_][v0_ + 2], sf_[kb_][v0_ + 3], pb[w_], true);      \
      }                                                                                                    \
    }                                                                                                      \
    __builtin_amdgcn_s_setprio(1);                                                                         \
    _Pragma("unroll") for (int j_ = 0; j_ < NPV; ++j_) {                                                   \
      const v4i a0_ = *reinterpret_cast<const v4i*>(vt_ + vo0 + j_ * 32 * BN);                             \
      const v4i a1_ = *reinterpret_cast<const v4i*>(vt_ + vo1 + j_ * 32 * BN);                             \
      const v8i va_ = {a0_[0], a0_[1], a0_[2], a0_[3], a1_[0], a1_[1], a1_[2], a1_[3]};                    \
      o[j_] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va_, pb, o[j_], 0, 0, 0, 0, 0, 0);           \
    }                                                                                                      \
    __builtin_amdgcn_s_setprio(0);                                                                         \
    next_ = sfail_ ? PASS_EXACT : (slow_ ? PASS_REDO : PASS_NONE);                                         \
  } while (0)

  // The tile's passes: one, or more when a speculative pass does not stand or some lane of the wave moves its max
  // at block 1 (the body sets next_: speculative -> exact -> redo, each at most once).  The
  // memory clobber keeps the LDS operand reads inside the loop, and the tile's mask word and bias values pass through
  // empty asm statements on every pass so that nothing derived from them (32 bit masks, 32 scaled biases) is hoisted
  // out of the loop and held across the whole body.
#define SAGE_TILE_PASSES(T, MODE, MW, BW, WIDE)                                                            \
  do {                                                                                                     \
    int kind_ = (SPEC_OK && fastok) ? PASS_SPEC : PASS_EXACT;                                              \
    int next_ = PASS_NONE;                                                                                 \
    _Pragma("nounroll") for (;;) {                                                                         \
      asm volatile("" ::: "memory");                                                                       \
      uint32_t mwp_ = (MW);                                                                                \
      if ((MODE) == 2) asm volatile("" : "+v"(mwp_));                                                      \
      if ((MODE) == 3) asm volatile("" : "+v"((BW)[0]), "+v"((BW)[1]), "+v"((BW)[2]), "+v"((BW)[3]));      \
      SAGE_TILE(T, MODE, mwp_, BW, kind_, WIDE);                                                           \
      if (next_ == PASS_NONE) break;                                                                       \
      kind_ = next_;                                                                                       \
    }                                                                                                      \
  } while (0)

  // Tiles before `t_mask` need no key mask for any row of this wave: they end below Skv and (causal) below the
  // wave's first row's diagonal.  The remaining tiles (at most three) run the masked variant.  The direct loads
  // are asynchronous writes to LDS the compiler does not track, hence the explicit vmcnt waits before barriers.
  int t_mask = Skv / BN;
  if (CAUSAL) t_mask = min(t_mask, max(0, (q0 + off + 1) / BN));
  t_mask = min(t_mask, t_hi);
  // QK accumulators start at the bits of c = fp32(1 / (2 pi)) (0x3E22F983, which the compiler encodes as the
  // MFMA's inline constant): the int32 sum read as fp32 is c + S * 2^-26, exactly; unseeded kernels start at 0
  v16i seed16;
#pragma unroll
  for (int v = 0; v < 16; ++v) seed16[v] = (int)SEED_BITS;
  // A split key range after the first starts from the running max that one online softmax over every key has after
  // the sequence's first tile (block 0 sets it, block 1 moves it by the lazy rule), instead of from -inf: the
  // reference's max almost never moves after its first tile, so the range then forms the same probabilities, E4M3
  // bytes and rescale decisions as the reference's walk (make_sage_r2.py:141-253) and its merge weight is l alone.
  // The first tile's K goes into the buffer the loop fills last (free until the loop's first prefetch), beside the
  // range's first tile(s); the dense split tiles are non-causal and unmasked and have at least 4 full key tiles.
  const bool seed_split = !MASK && !VARLEN && split && t_lo > 0;
  constexpr int SEED_BUF_OFS = NBUF - 1;  // buffer (t_lo + NBUF - 1) % NBUF
  if (seed_split) {
    const int8_t* kb_ = kbase;
    asm volatile("" : "+s"(kb_));
    uint8_t* dst_ = smem[(t_lo + SEED_BUF_OFS) % NBUF];
#pragma unroll
    for (int j = 0; j < KLOADS; ++j) {
      asm volatile("" : "+v"(koff[j]));
      copy16_to_lds(kb_ + koff[j], dst_ + (wave * KLOADS + j) * 1024);
    }
  }
  if (MASK && mseed_tile >= 0) {
    // The mask variant's seed: the block's first visited tile runs through the tile body of the wave's class (which
    // sets m as the walk's first tile does, the mask and an additive bias included), then its l and O are dropped.
    // It runs before the range's first tile is issued, which may reuse its buffer.
    const int ts = mseed_tile;
    SAGE_ISSUE_TILE(ts, ts % NBUF);
    const int cs = mcls[ts];
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (cs == 1) {
      SAGE_TILE_PASSES(ts, 0, 0u, bw_none, wide);
    } else if (cs == 2) {
      const uint32_t mw = load_global_u32(mbase + (moff + 8u * (uint32_t)ts));
      SAGE_TILE_PASSES(ts, 2, mw, bw_none, wide);
    } else if (cs == 3) {
      v4i bias_w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) bias_w[i] = load_global_v4i(bbase + (boff + 128u * (uint32_t)ts + 16u * i));
      SAGE_TILE_PASSES(ts, 3, 0u, bias_w, wide);
    }
    l = 0.0f;
#pragma unroll
    for (int i = 0; i < NPV; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[i][v] = 0.0f;
    __syncthreads();
  }
  // the first tile (and, with three buffers, the second) in flight; wait for the first
  if (t_lo < t_hi) SAGE_ISSUE_TILE(t_lo, t_lo % NBUF);
  const bool two_ahead = NBUF == 3 && t_lo + 1 < t_hi;
  if (two_ahead) SAGE_ISSUE_TILE(t_lo + 1, (t_lo + 1) % NBUF);
  if (seed_split) {
    // the first tile's K loads were issued before both tiles' loads
    if constexpr (NBUF == 3) {
      if (two_ahead)
        wait_vmcnt<2 * LPT>();
      else
        wait_vmcnt<LPT>();
    } else {
      wait_vmcnt<LPT>();
    }
    tile_barrier();
    const uint8_t* kt0 = smem[(t_lo + SEED_BUF_OFS) % NBUF];
    v16i s0, s1;
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      const v4i k0_ = *reinterpret_cast<const v4i*>(kt0 + ko[i]);
      const v4i k1_ = *reinterpret_cast<const v4i*>(kt0 + ko[i] + 32 * D);
      s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k0_, qa[i], i == 0 ? seed16 : s0, 0, 0, 0);
      s1 = i == 0 ? mfma_i8_seeded<SEEDED>(k1_, qa[i]) : __builtin_amdgcn_mfma_i32_32x32x32_i8(k1_, qa[i], s1, 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    // the two 32-key blocks' maxima in m's units (as the exact pass takes them)
    float mxh;
    if (SEEDED) {
      int mi0 = s0[0], mi1 = s1[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) {
        mi0 = max(mi0, s0[v]);
        mi1 = max(mi1, s1[v]);
      }
      mxh = __int_as_float(halves_max_i32(mi0, mi1));
    } else {
      float mx0 = (float)s0[0], mx1 = (float)s1[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) {
        mx0 = fmaxf(mx0, (float)s0[v]);
        mx1 = fmaxf(mx1, (float)s1[v]);
      }
      mxh = halves_max_f32(mx0, mx1);
    }
    const float ksh = hf ? ksb[1] : ksb[0];
    const float bmh = SEEDED ? (mxh - SEED_F) * ksh : mxh * ksh;
    float bm0, bm1;
    halves_split_f32(bmh, bm0, bm1);
    // from m = -inf block 0 always sets the max (its keys are all visible); block 1 moves it by the lazy rule
    const float mc1 = fmaxf(bm0, bm1);
    m = (mc1 - bm0) * cl > 8.0f ? mc1 : bm0;
    negm = 0.0f - cl * m;
    if (SPEC_OK) fastok = true;
  }
  if (two_ahead)
    wait_vmcnt<LPT>();
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  tile_barrier();
  int t = t_lo;
  if (MASK) {
    // per wave and tile: skip (class 0), the mask-free body (1) or the bit-masked body (2).  Runs of tiles of
    // classes 0 / 1 and runs of class 2 go through two loops with one tile body each (one loop holding both bodies
    // spills); each iteration of either ends in the workgroup barrier of its tile, and s_barrier counts waves, not
    // program locations, so the waves of a workgroup may sit in different loops.  The class of the next tile
    // (scalar) and, inside a run of class 2, the lane's mask word of the next tile are loaded one iteration ahead, so
    // the end-of-tile wait for the direct loads covers them and no wait inside a tile waits for the next tile.
    int c_nxt = t < t_hi ? mcls[t] : 0;
    while (t < t_hi) {
      for (; t < t_hi && c_nxt < 2; ++t) {
        const int c_cur = c_nxt;
        if (t + 1 < t_hi) {
          c_nxt = mcls[t + 1];
          SAGE_ISSUE_TILE(t + 1, (t + 1) & 1);
        }
        if (c_cur == 1) SAGE_TILE_PASSES(t, 0, 0u, bw_none, wide);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      }
      if (t < t_hi && c_nxt == 2) {  // a run of class 2 (its first word is waited for once)
        const uint8_t* mb_ = mbase;
        asm volatile("" : "+s"(mb_));
        uint32_t mw_cur = load_global_u32(mb_ + (moff + 8u * (uint32_t)t));
        // the uses below make the compiler's own waits for the words fall where the words are known to be complete
        // (here, and after the end-of-tile wait), not inside the next tile
        asm volatile("" ::"v"(mw_cur));
        for (; t < t_hi && c_nxt == 2; ++t) {
          uint32_t mw_nxt = 0u;
          if (t + 1 < t_hi) {
            mw_nxt = load_global_u32(mb_ + (moff + 8u * (uint32_t)(t + 1)));
            c_nxt = mcls[t + 1];
            SAGE_ISSUE_TILE(t + 1, (t + 1) & 1);
          }
          SAGE_TILE_PASSES(t, 2, mw_cur, bw_none, wide);
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          asm volatile("" ::"v"(mw_nxt));
          __syncthreads();
          mw_cur = mw_nxt;
        }
      }
      // a run of class 3 (additive mask): the lane's 64 bytes of bias values of the tile are loaded before the next
      // tile's direct loads, which are always issued here (the last iteration reloads its own tile into the idle
      // buffer), so the wait for the values counts the direct loads behind them and does not wait for them
      for (; t < t_hi && c_nxt == 3; ++t) {
        const uint8_t* bb_ = bbase;
        asm volatile("" : "+s"(bb_));
        v4i bias_w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) bias_w[i] = load_global_v4i(bb_ + (boff + 128u * (uint32_t)t + 16u * i));
        const int tn_ = min(t + 1, t_hi - 1);
        c_nxt = mcls[tn_];
        SAGE_ISSUE_TILE(tn_, (t + 1) & 1);
        SAGE_TILE_PASSES(t, 3, 0u, bias_w, wide);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      }
    }
  } else {
    // tile t + NBUF - 1 goes into the buffer tile t - 1 used, which every wave left at the last barrier; the end of
    // tile t waits for tile t + 1 (all but the LPT loads of tile t + 2 when those were issued: loads complete in order)
    constexpr int PF = NBUF - 1;
    // the mask-free loop in two copies, so that its tiles carry no test of `wide`
#define SAGE_MASK_FREE_LOOP(WIDE)                                                                          \
    for (; t < t_mask; ++t) {                                                                              \
      const bool ahead = t + PF < t_hi;                                                                    \
      if (ahead) SAGE_ISSUE_TILE(t + PF, (t + PF) % NBUF);                                                 \
      SAGE_TILE_PASSES(t, 0, 0u, bw_none, WIDE);                                                           \
      if (PF == 2 && ahead) wait_vmcnt<LPT>();                                                             \
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                                                \
      tile_barrier();                                                                                      \
    }
    if (wide) {
      SAGE_MASK_FREE_LOOP(true);
    } else {
      SAGE_MASK_FREE_LOOP(false);
    }
#undef SAGE_MASK_FREE_LOOP
    for (; t < t_hi; ++t) {
      const bool ahead = t + PF < t_hi;
      if (ahead) SAGE_ISSUE_TILE(t + PF, (t + PF) % NBUF);
      SAGE_TILE_PASSES(t, 1, 0u, bw_none, wide);
      if (PF == 2 && ahead) wait_vmcnt<LPT>();
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      tile_barrier();
    }
  }
#undef SAGE_ISSUE_TILE
#undef SAGE_TILE
#undef SAGE_TILE_PASSES

  // ---- epilogue ----
  const float lt = add_xor32_f32(l);
  if (split) {
    // partial state of this key range (workspace layout at ws_ml_offset), merged by attn_merge_kernel
    const int q = wave * 32 + ln;
    // A range that starts from the seeded max may hold only probabilities far below it, so l can be tiny (down to
    // subnormal, with every E4M3 byte 0 and O = 0): below 2^-64 both l and O are scaled by 2^64 (exact) before the
    // reciprocal, which then stays finite; l and O of order 1 and above are used as they are.
    const float ls = lt < 0x1p-64f ? 0x1p64f : 1.0f;
    const float rl = lt > 0.0f ? 1.0f / (lt * ls) : 0.0f;  // a range in which the row sees no key stores 0
    uint16_t* po = reinterpret_cast<uint16_t*>(part) + ((int64_t)unit * ATT_BM + q) * D;
#pragma unroll
    for (int i = 0; i < NPV; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t h0 = f32_to_f16_bits((o[i][4 * g + 0] * ls) * rl), h1 = f32_to_f16_bits((o[i][4 * g + 1] * ls) * rl);
        const uint32_t h2 = f32_to_f16_bits((o[i][4 * g + 2] * ls) * rl), h3 = f32_to_f16_bits((o[i][4 * g + 3] * ls) * rl);
        *reinterpret_cast<uint2*>(po + 32 * i + 8 * g + 4 * hf) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
      }
    const int64_t units = (int64_t)(total - n_full) * chunks;
    if (hf == 0)
      reinterpret_cast<float2*>(reinterpret_cast<uint8_t*>(part) + ws_ml_offset(units, D))[(int64_t)unit * ATT_BM + q] =
          make_float2(m * SSCALE, lt);  // m in S * ks units, as the merge kernel's cl expects
    return;
  }
  // The lane's V scales (its 4 * NPV groups of 4 channels), every load issued before the first is used: one round
  // trip instead of one per channel block.  VS rows hold D channels, so the loads stay in bounds for head_dim 96 too.
  const float* vsr = vs + (int64_t)bhk * D;
  v4f sc[NPV][4];
#pragma unroll
  for (int i = 0; i < NPV; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) sc[i][g] = *reinterpret_cast<const v4f*>(vsr + 32 * i + 8 * g + 4 * hf);
  const float inv = lt > 0.0f ? (1.0f / 448.0f) / lt : 0.0f;  // a row without any visible key is written as 0
  if (qvalid) {
    uint16_t* orow = obase + (int64_t)qrow * oss + h * osh;
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      if (32 * i >= dout) break;  // head_dim 96: the zero-padded channels are not written
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = 32 * i + 8 * g + 4 * hf;
        const v4f sc4 = sc[i][g];
        const uint32_t e0 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 0] * inv) * sc4[0]);
        const uint32_t e1 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 1] * inv) * sc4[1]);
        const uint32_t e2 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 2] * inv) * sc4[2]);
        const uint32_t e3 = f32_to_out_bits<OUT_DT>((o[i][4 * g + 3] * inv) * sc4[3]);
        *reinterpret_cast<uint2*>(orow + c) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
      }
    }
    if (!VARLEN && lse != nullptr && hf == 0) {
      // sum_j exp(logit_ij) = 2^(cl * m) * l_total, so lse = ln2 * (cl * m + log2(l_total))
      lse[qrow0 + qrow] = 0.69314718055994531f * (cl * m + __log2f(lt));
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// Merge of split tiles: one thread per (split tile s, row r, 4-channel group c), consecutive threads on consecutive
// groups of a row, so partial reads and output writes are contiguous; every partial load of a thread is issued before
// the first is used.  With M = max_i m_i over the chunks, W_i = 2^((m_i - M) * cl) * l_i, L = sum_i W_i and
// O = sum_i W_i * fp16(O_i / l_i) (float32, chunk order), the output is (O * ((1/448) / L)) * VS and
// lse = ln2 * (cl * M + log2 L), the epilogue of an unsplit tile.  grid = n_split * 128 * (D / 4) / 256 blocks of 256 threads.
// ------------------------------------------------------------------------------------------------------------------
template <int D, int OUT_DT>
__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ part, const float* __restrict__ qs,
                                                         const float* __restrict__ vs, uint16_t* __restrict__ out,
                                                         int64_t osb, int64_t oss, int64_t osh,
                                                         float* __restrict__ lse, int H, int Hkv, int Sq, int q_tiles,
                                                         int n_full, int n_split, int chunks, float c0, int dout) {
  constexpr int NG = D / 4;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int cg = idx % NG;
  if (4 * cg >= dout) return;  // head_dim 96: padding channels
  const int q = (idx / NG) % ATT_BM;
  const int s = idx / (NG * ATT_BM);
  const int logical = n_full + s;
  const int bh = logical / q_tiles, qt = logical % q_tiles;
  const int qrow = qt * ATT_BM + q;
  if (qrow >= Sq) return;
  const int b = bh / H, h = bh % H;
  const int bhk = b * Hkv + h / (H / Hkv);
  const int64_t units = (int64_t)n_split * chunks, unit0 = (int64_t)s * chunks;
  const float2* ml =
      reinterpret_cast<const float2*>(reinterpret_cast<const uint8_t*>(part) + ws_ml_offset(units, D)) + unit0 * ATT_BM + q;
  const uint16_t* po = reinterpret_cast<const uint16_t*>(part) + (unit0 * ATT_BM + q) * D + 4 * cg;
  // the row's Q scale and the group's V scales first, so that every load of the thread is in flight at once (loaded
  // after the merge arithmetic, the V scales cost a second round trip)
  const float qsr = qs[(int64_t)bh * Sq + qrow];
  const v4f sc4 = *reinterpret_cast<const v4f*>(vs + (int64_t)bhk * D + 4 * cg);
  float2 e[ATT_MAX_CHUNKS];
  uint2 oi[ATT_MAX_CHUNKS];
#pragma unroll
  for (int i = 0; i < ATT_MAX_CHUNKS; ++i) {
    if (i < chunks) {
      e[i] = ml[i * ATT_BM];
      oi[i] = *reinterpret_cast<const uint2*>(po + (int64_t)i * ATT_BM * D);
    }
  }
  const float cl = c0 * qsr;
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < ATT_MAX_CHUNKS; ++i)
    if (i < chunks) M = fmaxf(M, e[i].x);
  float L = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < ATT_MAX_CHUNKS; ++i) {
    if (i < chunks) {
      // chunk weight times its l; a range in which the row sees no key (l = 0, m = -inf) weighs 0
      const float w = e[i].y > 0.0f ? __builtin_amdgcn_exp2f((e[i].x - M) * cl) * e[i].y : 0.0f;
      L = L + w;
      acc.x = acc.x + w * f16_lo(oi[i].x);
      acc.y = acc.y + w * f16_hi(oi[i].x);
      acc.z = acc.z + w * f16_lo(oi[i].y);
      acc.w = acc.w + w * f16_hi(oi[i].y);
    }
  }
  const float inv = L > 0.0f ? (1.0f / 448.0f) / L : 0.0f;  // a row without any visible key is written as 0
  const uint32_t e0 = f32_to_out_bits<OUT_DT>((acc.x * inv) * sc4[0]);
  const uint32_t e1 = f32_to_out_bits<OUT_DT>((acc.y * inv) * sc4[1]);
  const uint32_t e2 = f32_to_out_bits<OUT_DT>((acc.z * inv) * sc4[2]);
  const uint32_t e3 = f32_to_out_bits<OUT_DT>((acc.w * inv) * sc4[3]);
  uint16_t* orow = out + b * osb + (int64_t)qrow * oss + h * osh;
  *reinterpret_cast<uint2*>(orow + 4 * cg) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
  if (lse != nullptr && cg == 0) lse[(int64_t)bh * Sq + qrow] = 0.69314718055994531f * (cl * M + __log2f(L));
}

// ------------------------------------------------------------------------------------------------------------------
// Work plan.  A launch of n_tiles query tiles runs in rounds of `slots` = CUs x resident workgroups per CU.  When the
// last round is short (rem = n_tiles mod slots tiles), its tiles run at a fraction of the chip's throughput: the
// plan splits the key range of those rem tiles into chunks = slots / rem parts (at most 16, at least 4 key tiles
// each) so that the last round fills the chip again, and a merge kernel combines the parts.  Causal tiles are
// never split.
// ------------------------------------------------------------------------------------------------------------------
struct AttnPlan {
  int n_tiles, n_full, chunks;
  int64_t workspace;  // bytes of partial state
};

static int device_cus(int* cus) {
  static int cache[64] = {0};
  int dev = 0;
  SAGE_HIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
  if (dev >= 0 && dev < 64 && cache[dev] > 0) {
    *cus = cache[dev];
    return SAGE_OK;
  }
  int n = 0;
  SAGE_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
  if (dev >= 0 && dev < 64) cache[dev] = n;
  *cus = n;
  return SAGE_OK;
}

// HD: head dim (the kernel's template argument; its layouts have layout_dim(HD) channels)
template <int HD, bool CAUSAL, int OUT_DT>
static int resident_blocks(int* per_cu) {
  static int cache = 0;
  if (cache == 0) {
    int n = 0;
    SAGE_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_kernel<HD, CAUSAL, OUT_DT, false>, ATT_THREADS, 0),
                   "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    cache = n;
  }
  *per_cu = cache;
  return SAGE_OK;
}

template <int HD, bool CAUSAL, int OUT_DT>
static int make_plan(int B, int H, int Sq, int Skv, AttnPlan* p) {
  constexpr int D = layout_dim(HD);
  const int q_tiles = (Sq + ATT_BM - 1) / ATT_BM;
  p->n_tiles = B * H * q_tiles;
  p->n_full = p->n_tiles;
  p->chunks = 1;
  p->workspace = 0;
  if (CAUSAL) return SAGE_OK;
  int cus = 0, per_cu = 0, rc;
  if ((rc = device_cus(&cus))) return rc;
  if ((rc = resident_blocks<HD, CAUSAL, OUT_DT>(&per_cu))) return rc;
  const int slots = cus * per_cu;
  if (slots <= 0) return SAGE_OK;
  const int rem = p->n_tiles % slots;
  if (rem == 0) return SAGE_OK;
  const int kv_tiles = (Skv + ATT_BN - 1) / ATT_BN;
  const int chunks = min(min(slots / rem, kv_tiles / 4), ATT_MAX_CHUNKS);
  if (chunks < 2) return SAGE_OK;
  p->n_full = p->n_tiles - rem;
  p->chunks = chunks;
  p->workspace = ws_bytes((int64_t)rem * chunks, D);
  return SAGE_OK;
}

// c0 = log2(e) / sqrt(head_dim) with the kernel's built-in sm_scale (other scales are folded into QS)
static float logit_scale_base(int head_dim) { return (float)((1.0 / __builtin_sqrt((double)head_dim)) * 1.4426950408889634); }

// HD: head dim (64, 96, 128, 256); D = layout_dim(HD) channels of the intermediates (96 runs on the 128-channel
// layout); hd == HD, the output channels
template <int HD, bool CAUSAL, int OUT_DT>
static int launch_attn(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                       const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, float* lse, int B, int H,
                       int Hkv, int Sq, int Skv, int hd, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  constexpr int D = layout_dim(HD);
  AttnPlan p;
  int rc;
  if (workspace == nullptr) {
    const int q_tiles = (Sq + ATT_BM - 1) / ATT_BM;
    p.n_tiles = p.n_full = B * H * q_tiles;
    p.chunks = 1;
    p.workspace = 0;
  } else {
    if ((rc = make_plan<HD, CAUSAL, OUT_DT>(B, H, Sq, Skv, &p))) return rc;
    SAGE_REQUIRE(workspace_bytes >= p.workspace, "sage_attn_fwd: workspace of %lld bytes, the plan needs %lld",
                 (long long)workspace_bytes, (long long)p.workspace);
    SAGE_REQUIRE(((uintptr_t)workspace & 255u) == 0, "sage_attn_fwd: workspace must be 256-byte aligned");
  }
  const int q_tiles = (Sq + ATT_BM - 1) / ATT_BM;
  const int n_split = p.n_tiles - p.n_full;
  const int blocks = p.n_full + n_split * p.chunks;
  const float c0 = logit_scale_base(hd);
  uint16_t* o = static_cast<uint16_t*>(out);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL((attn_kernel<HD, CAUSAL, OUT_DT, false>), dim3(blocks), dim3(ATT_THREADS), 0, st, q8, qs, k8, ks, v8t,
                     vs, o, osb, oss, osh, lse, H, Hkv, Sq, Skv, kv_pad(Skv), q_tiles, p.n_tiles, p.n_full, p.chunks,
                     part, c0, hd, VarlenTiles{}, MaskTabs{}, nullptr, nullptr, nullptr, nullptr);
  if (n_split > 0) {
    if ((rc = check_launch("attention launch"))) return rc;
    hipLaunchKernelGGL((attn_merge_kernel<D, OUT_DT>), dim3(n_split * (ATT_BM * D / 4 / 256)), dim3(256), 0, st,
                       part, qs, vs, o, osb, oss, osh, lse, H, Hkv, Sq, q_tiles, p.n_full, n_split, p.chunks, c0, hd);
  }
  return check_launch("attention launch");
}

static int check_attn_shape(int B, int H, int Hkv, int Sq, int Skv, int D, int causal, const char* who) {
  SAGE_REQUIRE(B > 0 && H > 0 && Hkv > 0 && Sq > 0 && Skv > 0, "%s: sizes must be positive", who);
  SAGE_REQUIRE(H % Hkv == 0, "%s: heads %d not a multiple of kv heads %d", who, H, Hkv);
  if (!head_dim_ok(D)) return fail(SAGE_ERR_UNSUPPORTED, "%s: head_dim %d (supported 64, 96, 128, 256)", who, D);
  if (causal && Sq > Skv) return fail(SAGE_ERR_UNSUPPORTED, "%s: causal attention needs q_len <= kv_len", who);
  SAGE_REQUIRE((int64_t)B * H * ((Sq + ATT_BM - 1) / ATT_BM) * ATT_MAX_CHUNKS < (1ll << 31), "%s: too many query tiles",
               who);
  SAGE_REQUIRE((int64_t)layout_dim(D) * kv_pad(Skv) < (1ll << 31), "%s: kv_len %d too long", who, Skv);
  return SAGE_OK;
}

// dispatch on the head dim (checked by the caller to be 64, 96, 128 or 256)
#define SAGE_ATTN_DISPATCH_HD(HDV, CAUSAL, BF, FN, ...)                                                         \
  ((CAUSAL) ? ((BF) ? FN<HDV, true, DT_BF16>(__VA_ARGS__) : FN<HDV, true, DT_F16>(__VA_ARGS__))                \
            : ((BF) ? FN<HDV, false, DT_BF16>(__VA_ARGS__) : FN<HDV, false, DT_F16>(__VA_ARGS__)))
#define SAGE_ATTN_DISPATCH(HD, CAUSAL, BF, FN, ...)                                                             \
  ((HD) == 64    ? SAGE_ATTN_DISPATCH_HD(64, CAUSAL, BF, FN, __VA_ARGS__)                                       \
   : (HD) == 96  ? SAGE_ATTN_DISPATCH_HD(96, CAUSAL, BF, FN, __VA_ARGS__)                                       \
   : (HD) == 128 ? SAGE_ATTN_DISPATCH_HD(128, CAUSAL, BF, FN, __VA_ARGS__)                                      \
                 : SAGE_ATTN_DISPATCH_HD(256, CAUSAL, BF, FN, __VA_ARGS__))

int attn_plan_impl(int B, int H, int Sq, int Skv, int D, int causal, int* n_full, int* chunks, int64_t* ws) {
  int rc = check_attn_shape(B, H, H, Sq, Skv, D, causal, "sage_attn_plan");
  if (rc) return rc;
  AttnPlan p;
  // the plan depends on the kernel's occupancy, which is the same for both output dtypes
  if ((rc = SAGE_ATTN_DISPATCH(D, causal, true, make_plan, B, H, Sq, Skv, &p))) return rc;
  if (n_full) *n_full = p.n_full;
  if (chunks) *chunks = p.chunks;
  if (ws) *ws = p.workspace;
  return SAGE_OK;
}

// Every argument check of the attention step: sage_forward runs it before its first launch as well.
int attn_args_check(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                    const float* vs, const void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv,
                    int Sq, int Skv, int D, int causal, int out_dtype, const char* who) {
  int rc = check_attn_shape(B, H, Hkv, Sq, Skv, D, causal, who);
  if (rc) return rc;
  if (out_dtype != SAGE_DTYPE_BF16 && out_dtype != SAGE_DTYPE_F16)
    return fail(SAGE_ERR_UNSUPPORTED, "%s: out dtype code %d", who, out_dtype);
  SAGE_REQUIRE(q8 && qs && k8 && ks && v8t && vs && out, "%s: a pointer argument is NULL", who);
  SAGE_REQUIRE(aligned16(q8) && aligned16(k8) && aligned16(v8t) && aligned16(vs) && aligned16(out),
               "%s: q8 / k8 / v8t / vs / out must be 16-byte aligned", who);
  SAGE_REQUIRE(osb % 8 == 0 && oss % 8 == 0 && osh % 8 == 0 && osb >= 0 && oss >= 0 && osh >= 0,
               "%s: out strides must be non-negative multiples of 8 elements", who);
  return SAGE_OK;
}

int attn_impl(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t, const float* vs,
              void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq, int Skv, int D,
              int causal, int out_dtype, float* lse, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = attn_args_check(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, causal, out_dtype,
                           "sage_attn_fwd");
  if (rc) return rc;
  return SAGE_ATTN_DISPATCH(D, causal, out_dtype == SAGE_DTYPE_BF16, launch_attn, q8, qs, k8, ks, v8t, vs, out, osb,
                            oss, osh, lse, B, H, Hkv, Sq, Skv, D, workspace, workspace_bytes, (hipStream_t)stream);
}

}  // namespace sage

namespace sage {

template <int HD, bool CAUSAL, int OUT_DT>
static int launch_attn_varlen(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks,
                              const uint8_t* v8t, const float* vs, void* out, int64_t oss, int64_t osh, int H, int Hkv,
                              int TQ, int TKP, int hd, int n_blocks, VarlenTiles vt, hipStream_t st) {
  hipLaunchKernelGGL((attn_kernel<HD, CAUSAL, OUT_DT, true>), dim3(n_blocks), dim3(ATT_THREADS), 0, st, q8, qs, k8, ks,
                     v8t, vs, static_cast<uint16_t*>(out), (int64_t)0, oss, osh, nullptr, H, Hkv, TQ, 0, TKP, 0,
                     n_blocks, n_blocks, 1, nullptr, logit_scale_base(hd), hd, vt, MaskTabs{}, nullptr, nullptr,
                     nullptr, nullptr);
  return check_launch("varlen attention launch");
}

// Validation is done by the caller (sage_forward_varlen).  n_blocks = entries of the tile table.
int attn_varlen_impl(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                     const float* vs, void* out, int64_t oss, int64_t osh, int H, int Hkv, int TQ, int TKP, int D,
                     int causal, int out_dtype, int n_blocks, const void* tiles, const int* cu_q, const int* cu_k,
                     const int* kp, void* stream) {
  const VarlenTiles vt{static_cast<const int4*>(tiles), cu_q, cu_k, kp};
  return SAGE_ATTN_DISPATCH(D, causal, out_dtype == SAGE_DTYPE_BF16, launch_attn_varlen, q8, qs, k8, ks, v8t, vs, out,
                            oss, osh, H, Hkv, TQ, TKP, D, n_blocks, vt, (hipStream_t)stream);
}

// Masked attention (the mask variant of the kernel; validation by the caller, sage_forward_masked).  The plan is
// the dense non-causal one (sage_attn_plan with causal = 0; the causal flag lives in the mask bits), so callers can
// query it; the mask variant's occupancy is never below the dense kernel's.
template <int HD, bool CAUSAL, int OUT_DT>
static int plan_mask(int B, int H, int Sq, int Skv, AttnPlan* p) {
  return make_plan<HD, false, OUT_DT>(B, H, Sq, Skv, p);
}

int attn_mask_plan_impl(int B, int H, int Sq, int Skv, int D, int64_t* ws) {
  AttnPlan p;
  int rc = SAGE_ATTN_DISPATCH(D, false, true, plan_mask, B, H, Sq, Skv, &p);
  if (rc) return rc;
  *ws = p.workspace;
  return SAGE_OK;
}

template <int HD, bool CAUSAL, int OUT_DT>
static int launch_attn_mask(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                            const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv,
                            int Sq, int Skv, int hd, MaskTabs mt, void* workspace, hipStream_t st) {
  constexpr int D = layout_dim(HD);
  AttnPlan p;
  int rc;
  if ((rc = plan_mask<HD, false, OUT_DT>(B, H, Sq, Skv, &p))) return rc;
  const int q_tiles = (Sq + ATT_BM - 1) / ATT_BM;
  const int n_split = p.n_tiles - p.n_full;
  const int blocks = p.n_full + n_split * p.chunks;
  const float c0 = logit_scale_base(hd);
  uint16_t* o = static_cast<uint16_t*>(out);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL((attn_kernel<HD, false, OUT_DT, false, true>), dim3(blocks), dim3(ATT_THREADS), 0, st, q8, qs, k8,
                     ks, v8t, vs, o, osb, oss, osh, nullptr, H, Hkv, Sq, Skv, kv_pad(Skv), q_tiles, p.n_tiles,
                     p.n_full, p.chunks, part, c0, hd, VarlenTiles{}, mt, mt.bits, mt.cls, mt.range, mt.bias);
  if (n_split > 0) {
    if ((rc = check_launch("masked attention launch"))) return rc;
    hipLaunchKernelGGL((attn_merge_kernel<D, OUT_DT>), dim3(n_split * (ATT_BM * D / 4 / 256)), dim3(256), 0, st,
                       part, qs, vs, o, osb, oss, osh, nullptr, H, Hkv, Sq, q_tiles, p.n_full, n_split, p.chunks, c0,
                       hd);
  }
  return check_launch("masked attention launch");
}

// workspace: at least attn_mask_plan_impl bytes (may be NULL when that is 0)
int attn_mask_impl(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                   const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv, int Sq,
                   int Skv, int D, int out_dtype, const MaskTabs* mt, void* workspace, void* stream) {
  return SAGE_ATTN_DISPATCH(D, false, out_dtype == SAGE_DTYPE_BF16, launch_attn_mask, q8, qs, k8, ks, v8t, vs, out,
                            osb, oss, osh, B, H, Hkv, Sq, Skv, D, *mt, workspace, (hipStream_t)stream);
}

}  // namespace sage

extern "C" int sage_attn_plan(int B, int H, int Sq, int Skv, int D, int causal, int* n_full, int* chunks,
                              int64_t* workspace_bytes) {
  sage::clear_error();
  return sage::attn_plan_impl(B, H, Sq, Skv, D, causal, n_full, chunks, workspace_bytes);
}

extern "C" int sage_attn_fwd(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, const uint8_t* v8t,
                             const float* vs, void* out, int64_t osb, int64_t oss, int64_t osh, int B, int H, int Hkv,
                             int Sq, int Skv, int D, int causal, int out_dtype, float* lse, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  sage::clear_error();
  return sage::attn_impl(q8, qs, k8, ks, v8t, vs, out, osb, oss, osh, B, H, Hkv, Sq, Skv, D, causal, out_dtype, lse,
                         workspace, workspace_bytes, stream);
}
