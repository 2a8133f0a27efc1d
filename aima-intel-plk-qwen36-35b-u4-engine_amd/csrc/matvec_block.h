// The batch-1 U4 matvec's block body (rows blk * BR .. +BR of one matrix),
// shared by the matvec kernels (u4_matvec.hip) and the LM head with top-k
// (lm_head.hip).
//
// Decode matvec: each row of K/2 packed bytes is split into 16-byte chunks
// (32 nibbles, always inside one quantization group because group % 32 == 0).
// A wave covers 64 chunks: one row at K=2048, four rows at K=512.  Every lane
// issues one 128-bit global load per row, unpacks in registers and reduces
// with two v_dot2_f32_f16 chains (see XChunk in common.h), then the row's
// segment is reduced across lanes.  Row groups are loaded before any compute
// so each wave keeps RG x 1 KB in flight; the block's scales and zero points
// (contiguous, its rows being consecutive) are staged through LDS.
#ifndef AIMA_MATVEC_BLOCK_H_
#define AIMA_MATVEC_BLOCK_H_

#include "common.h"

namespace aima {

// The tag of a stored logit: the launch number xor a hash of the value's
// bits.  A word of another launch, or other data under the region, passes
// only if its high half equals that function of its low half (the hash is a
// bijection of the bits, so exactly one low half matches a given high half).
__device__ __forceinline__ uint32_t logit_tag(uint32_t bits, uint32_t launch) {
  return launch ^ (bits * 0x9E3779B1u + 0x7F4A7C15u);
}

template <int KCH>
struct RowGeom {
  static constexpr int NC = KCH > 64 ? KCH / 64 : 1;  // chunks per lane per row
  static constexpr int SEG = KCH > 64 ? 64 : KCH;     // lanes per row
  static constexpr int RPI = 64 / SEG;                // rows per wave pass
  static constexpr int K = KCH * 32;
};

// The lane's activation chunks (chunk c = cl + i*SEG of f16 x) as raw
// 16-byte words; make_xchunk builds the dot-product operands once they land.
template <int KCH>
__device__ __forceinline__ void load_x_raw(const uint16_t* __restrict__ x, int cl,
                                           u32x4 (&xr)[RowGeom<KCH>::NC][4]) {
  using G = RowGeom<KCH>;
#pragma unroll
  for (int i = 0; i < G::NC; ++i) {
    const u32x4* p = reinterpret_cast<const u32x4*>(x + (int64_t)(cl + i * G::SEG) * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) xr[i][q] = p[q];
  }
}

template <int KCH>
__device__ __forceinline__ void build_x_chunks(const u32x4 (&xr)[RowGeom<KCH>::NC][4],
                                               XChunk (&xc)[RowGeom<KCH>::NC]) {
  using G = RowGeom<KCH>;
#pragma unroll
  for (int i = 0; i < G::NC; ++i) {
    uint32_t w[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      w[4 * q + 0] = xr[i][q][0];
      w[4 * q + 1] = xr[i][q][1];
      w[4 * q + 2] = xr[i][q][2];
      w[4 * q + 3] = xr[i][q][3];
    }
    make_xchunk(w, xc[i]);
  }
}

// Rows blk * BR .. +BR of one matrix (the body of every matvec block).
//
// Load order: the block's scales and zero points (contiguous: its rows are
// consecutive), then the activations, then the weights, with nothing waited
// for in between.  Loads complete in order, so staging the scales in LDS
// and building the activation operands waits only for those, while every
// weight load is still in flight.
//
// tagged (optional; used only where a wave pass covers one row, K >= 2048):
// the f32 result of row r is also stored as the 64-bit word {bits, logit_tag(bits, tag)} at
// tagged[r] (the LM head's fused top-k reads those).
template <int KCH, int RG>
__device__ __forceinline__ void matvec_block(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ qw,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zp,
    int64_t n, int group_log2, void* __restrict__ y, int out_f32, int64_t blk,
    uint64_t* __restrict__ tagged = nullptr, uint32_t tag = 0) {
  using G = RowGeom<KCH>;
  constexpr int BR = 4 * RG * G::RPI;       // rows of the block (consecutive)
  constexpr int kMaxGroups = G::K / 32;     // groups per row at group 32
  // 32-bit words of scales / zero points per thread at the most groups
  constexpr int kSW = (BR * kMaxGroups / 2 + 255) / 256;
  constexpr int kZW = (BR * kMaxGroups / 8 + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[BR * kMaxGroups];
  __shared__ __attribute__((aligned(16))) uint8_t z_lds[BR * kMaxGroups / 2];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int seg = lane / G::SEG;
  const int cl = lane % G::SEG;
  const int groups = G::K >> group_log2;
  const uint32_t magic = u4_magic();

  const int64_t brow0 = blk * BR;
  const int64_t row0 = brow0 + (int64_t)wave * (RG * G::RPI);
  const int64_t rows_here = n - brow0 < BR ? n - brow0 : BR;
  const int nsc = (int)rows_here * groups;  // scales (and zero-point nibbles) of the block
  const int zbytes = (nsc + 1) / 2;
  const uint16_t* sblk = scale + brow0 * groups;
  const uint8_t* zblk = zp + (brow0 * groups >> 1);
  // 32-bit words where the block's runs are 4-byte aligned (always, for
  // 4-byte aligned arrays); the remainder element by element
  const bool s_words = (reinterpret_cast<uintptr_t>(sblk) & 3u) == 0;
  const bool z_words = (reinterpret_cast<uintptr_t>(zblk) & 3u) == 0;
  const int s_full = s_words ? nsc / 2 : 0, z_full = z_words ? zbytes / 4 : 0;
  uint32_t sw[kSW], zw[kZW];
#pragma unroll
  for (int j = 0; j < kSW; ++j) {
    const int i = tid + 256 * j;
    sw[j] = i < s_full ? reinterpret_cast<const uint32_t*>(sblk)[i] : 0u;
  }
#pragma unroll
  for (int j = 0; j < kZW; ++j) {
    const int i = tid + 256 * j;
    zw[j] = i < z_full ? reinterpret_cast<const uint32_t*>(zblk)[i] : 0u;
  }
  u32x4 xr[G::NC][4];
  load_x_raw<KCH>(x, cl, xr);
  // rows past n load row n - 1 instead (straight-line loads, no branch
  // around each); their results are never written
  u32x4 w[RG][G::NC];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int64_t row = row0 + r * G::RPI + seg;
    const int64_t rowc = row < n ? row : n - 1;
#pragma unroll
    for (int i = 0; i < G::NC; ++i) {
      const int c = cl + i * G::SEG;
      w[r][i] = load16_nt(qw + rowc * (G::K / 2) + (int64_t)c * 16);
    }
  }
#pragma unroll
  for (int j = 0; j < kSW; ++j) {
    const int i = tid + 256 * j;
    if (i < s_full) reinterpret_cast<uint32_t*>(s_lds)[i] = sw[j];
  }
#pragma unroll
  for (int j = 0; j < kZW; ++j) {
    const int i = tid + 256 * j;
    if (i < z_full) reinterpret_cast<uint32_t*>(z_lds)[i] = zw[j];
  }
  for (int t = 2 * s_full + tid; t < nsc; t += 256) s_lds[t] = sblk[t];
  for (int t = 4 * z_full + tid; t < zbytes; t += 256) z_lds[t] = zblk[t];
  XChunk xc[G::NC];
  build_x_chunks<KCH>(xr, xc);
  __syncthreads();
  // one row per wave pass: lane r < RG keeps the wave's row r and the wave
  // stores its RG consecutive results with one instruction
  float row_v = 0.f;
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int rl = wave * (RG * G::RPI) + r * G::RPI + seg;  // row within the block
    const int64_t row = brow0 + rl;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < G::NC; ++i) {
      const int c = cl + i * G::SEG;
      const int gi = rl * groups + ((c * 32) >> group_log2);
      const float sv = row < n ? h2f(s_lds[gi]) : 0.f;
      const uint32_t zv = row < n ? (uint32_t)(z_lds[gi >> 1] >> ((gi & 1) * 4)) & 0xfu : 0u;
      acc += u4_chunk_dot(w[r][i], xc[i], zv, sv, magic);
    }
    acc = segment_sum<G::SEG>(acc);
    if (G::RPI == 1) {
      row_v = lane == r ? acc : row_v;  // the sum is wave-uniform
    } else if (cl == 0 && row < n) {
      if (out_f32) {
        reinterpret_cast<float*>(y)[row] = acc;
      } else {
        reinterpret_cast<uint16_t*>(y)[row] = f2h(acc);
      }
    }
  }
  if (G::RPI == 1 && lane < RG) {
    const int64_t row = row0 + lane;
    if (row < n) {
      if (out_f32) {
        reinterpret_cast<float*>(y)[row] = row_v;
      } else {
        reinterpret_cast<uint16_t*>(y)[row] = f2h(row_v);
      }
      if (tagged) {
        // the logit with the launch number beside it, stored whole at device
        // scope (a reader on any XCD can tell it from an earlier launch's)
        const uint32_t bits = __builtin_bit_cast(uint32_t, row_v);
        __hip_atomic_store(&tagged[row], (uint64_t)bits | ((uint64_t)logit_tag(bits, tag) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

}  // namespace aima

#endif  // AIMA_MATVEC_BLOCK_H_
