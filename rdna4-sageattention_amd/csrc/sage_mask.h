// Attention masks (bool, or additive bf16 / fp16): the device work that turns a torch mask into the tables the
// attention kernel's mask variant reads (MaskTabs in sage_host.h).  It runs as extra workgroups of sage_forward's
// two quantization launches (no launch of its own): the bits, classes and bias values in the first, the
// per-workgroup tile ranges in the second, which stream order places after the first.
#pragma once

#include "sage_common.h"
#include "sage_host.h"

namespace sage {

// Everything the two kinds of mask workgroups need.  prep_blocks / range_blocks = 0: no mask work (the dense call).
struct MaskPrep {
  const void* mask;         // element (b, h, row, key) at mask + b*msb + h*msh + row*msq + key (element strides)
  int mdt;                  // SAGE_DTYPE_BOOL (nonzero byte = attend) or SAGE_DTYPE_BF16 / SAGE_DTYPE_F16 (additive)
  int64_t msb, msh, msq;
  int mh, mq, mg, nt, nrb;  // table extents (sage_mask.hip: mask_shape)
  int Sq, Skv, causal;
  int a4;                   // mask rows aligned to a run of 4 keys (4 bytes bool, 8 bytes 16-bit): one load per run
  uint32_t* bits;
  uint16_t* bias;           // 16-bit masks: the values of class-3 tiles, 32 per (row, tile, lane half), lane order
  int* cls;
  int2* range;
  int nrange;               // mb * mh * nrb
  int prep_blocks, range_blocks;
};

// One wave per (mask batch-head, 32-row group, tile); a block is 4 waves on 4 consecutive tiles.  Lane (row r =
// lane % 32 of the group, half hf = lane / 32) reads the 32 mask elements of its keys (8 runs of 4 consecutive keys:
// run j holds keys 64 t + 8 j + 4 hf + i at bits 4 j + i, values 4 j + i of the lane's bias entry).  Bool masks:
// a key is visible when its byte is nonzero.  16-bit (additive) masks: when its value is not -inf; the lane's keys
// are also "zero" (every value +-0) or "general" (some value neither 0 nor -inf).  Keys past kv_len and, causal,
// past the bottom-right diagonal are -inf.  Wave ballots give the class: 0 no row sees a key, 1 every key of every
// row visible with a zero bias, 2 visibility only (bool masks, or 16-bit values all 0 / -inf), 3 a general bias, whose
// values each lane then stores (-inf where masked).  Rows past q_len (and, for a mask without rows, every row but 0)
// count as neither seeing nor missing a key.  block < mb * mh * mg * ceil(nt / 4).
__device__ __forceinline__ void mask_prep_block(const MaskPrep& p, int block) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, hf = lane >> 5;
  const int ntb = (p.nt + 3) >> 2;
  const int t = (block % ntb) * 4 + wave;
  const int rest = block / ntb;
  const int g = rest % p.mg;
  const int mbh = rest / p.mg;
  if (t >= p.nt) return;  // the whole wave
  const int mbi = mbh / p.mh, mhi = mbh % p.mh;
  const int q = g * 32 + r;  // table row (mq == 1: row 0 only)
  const bool real = p.mq == 1 ? r == 0 : q < p.Sq;
  const int64_t entry = ((int64_t)mbh * p.mq + q) * p.nt + t;  // (row, tile) of the tables
  uint32_t w = 0;
  bool zero = true, general = false;
  uint32_t vals[16];  // 16-bit masks: the lane's 32 values, two per word, -inf where masked
  if (real) {
    const int lim = p.causal ? min(p.Skv - 1, q + (p.Skv - p.Sq)) : p.Skv - 1;  // last key the row may see
    const int k0 = t * 64 + 4 * hf;
    const int64_t rowoff = mbi * p.msb + mhi * p.msh + (int64_t)q * p.msq;
    if (p.mdt == SAGE_DTYPE_BOOL) {
      const uint8_t* row = static_cast<const uint8_t*>(p.mask) + rowoff;
      uint32_t b4[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kj = k0 + 8 * j;
        if (p.a4 && kj + 3 < p.Skv) {
          b4[j] = *reinterpret_cast<const uint32_t*>(row + kj);
        } else {
          b4[j] = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kj + i < p.Skv) b4[j] |= (uint32_t)row[kj + i] << (8 * i);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool vis = ((b4[j] >> (8 * i)) & 0xFFu) != 0 && k0 + 8 * j + i <= lim;
          w |= (uint32_t)vis << (4 * j + i);
        }
    } else {
      const uint16_t* row = static_cast<const uint16_t*>(p.mask) + rowoff;
      const uint16_t ninf = p.mdt == SAGE_DTYPE_BF16 ? 0xFF80u : 0xFC00u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kj = k0 + 8 * j;
        uint16_t e[4];
        if (p.a4 && kj + 3 < p.Skv) {
          const uint2 u = *reinterpret_cast<const uint2*>(row + kj);
          e[0] = (uint16_t)(u.x & 0xFFFFu);
          e[1] = (uint16_t)(u.x >> 16);
          e[2] = (uint16_t)(u.y & 0xFFFFu);
          e[3] = (uint16_t)(u.y >> 16);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) e[i] = kj + i < p.Skv ? row[kj + i] : ninf;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (k0 + 8 * j + i > lim) e[i] = ninf;
          const bool vis = e[i] != ninf;
          const bool z = (e[i] & 0x7FFFu) == 0;
          w |= (uint32_t)vis << (4 * j + i);
          zero = zero && z;
          general = general || (vis && !z);
        }
        vals[2 * j] = (uint32_t)e[0] | ((uint32_t)e[1] << 16);
        vals[2 * j + 1] = (uint32_t)e[2] | ((uint32_t)e[3] << 16);
      }
    }
    p.bits[entry * 2 + hf] = w;
  }
  const uint64_t any = __ballot(real && w != 0);
  const uint64_t all = __ballot(!real || (w == 0xFFFFFFFFu && zero));
  const uint64_t gen = __ballot(real && general);
  const int cls = any == 0 ? 0 : gen != 0 ? 3 : all == ~0ull ? 1 : 2;
  if (cls == 3 && real) {  // wave-uniform class
    uint4* dst = reinterpret_cast<uint4*>(p.bias + (entry * 2 + hf) * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(vals[4 * i], vals[4 * i + 1], vals[4 * i + 2], vals[4 * i + 3]);
  }
  if (lane == 0) p.cls[((int64_t)mbh * p.mg + g) * p.nt + t] = cls;
}

// One wave per (mask batch-head, 128-row block): the first and one past the last tile whose class is not 0 in any of
// the block's four 32-row groups (groups past the last one repeat it), (nt, 0) when there is none.  Lanes scan the
// 4 x nt classes with all their loads in flight, then a wave reduction.  block < ceil(nrange / 4).
__device__ __forceinline__ void mask_range_block(const MaskPrep& p, int block) {
  const int wid = block * 4 + (int)(threadIdx.x >> 6);
  if (wid >= p.nrange) return;  // the whole wave
  const int lane = threadIdx.x & 63;
  const int mbh = wid / p.nrb, rb = wid % p.nrb;
  int lo = p.nt, hi = -1;
  for (int i = lane; i < 4 * p.nt; i += 64) {
    const int g = min(rb * 4 + i / p.nt, p.mg - 1), t = i % p.nt;
    if (p.cls[((int64_t)mbh * p.mg + g) * p.nt + t] != 0) {
      lo = min(lo, t);
      hi = max(hi, t);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o));
    hi = max(hi, __shfl_xor(hi, o));
  }
  if (lane == 0) p.range[wid] = make_int2(lo, hi + 1);
}

}  // namespace sage
