// Grouped MoE prefill on gfx950.
//
// 1. Device schedule (three small launches): a stable counting sort of the
//    T*k (token, rank) assignments by expert.  Rows of one expert are ordered
//    by assignment index, the order of the reference's host
//    BuildGroupedSchedule (grouped_s8_u4_prefill_runtime.cpp:231-346), so the
//    schedule is deterministic and bit-comparable with the CPU restatement.
//    The scan also emits the list of 128-row M tiles (routed experts, then the
//    shared expert over all T tokens).
// 2. Grouped gate/up GEMM (MFMA v_mfma_f32_32x32x16_f16): per tile, the token
//    rows are gathered into LDS (double-buffered per 128-wide K group); each
//    wave dequantizes its own 64 weight rows (32 gate + the matching 32 up)
//    straight from HBM into MFMA B operands as exact f16 (q - z), runs 8
//    K-steps into a per-group accumulator and folds it into the f32 total
//    with the group's f16 scale.  The SwiGLU epilogue writes f16 [rows][I].
// 3. Grouped down GEMM, same structure over K = I, epilogue multiplies by the
//    router weight and writes f32 contributions [rows][H].
// 4. Combine: per token, the k contributions in rank order, plus the
//    sigmoid-gated shared row, plus the residual, rounded to f16.
//
// f16 rather than bf16 operands: the activations arrive as f16 and (q - z) is
// an integer in [-15, 15], so every MFMA product is exact and the only
// rounding besides f32 accumulation is the f16 SwiGLU output; MI355X runs
// dense f16 and bf16 MFMA at the same rate.
#include "common.h"

#include <math.h>

#include <algorithm>

namespace aima {

constexpr int kBM = 128;            // rows per M tile
constexpr int kSchedBlock = 1024;   // assignments per schedule block
constexpr int kLdsRowHalves = 136;  // 128 halves + 8 pad: 272-byte LDS rows
constexpr int kMaxExperts = 1024;

struct PrefillWs {
  uint32_t* err;
  int32_t* tile_count;
  int32_t* block_base;   // [nb][E]
  int32_t* offsets;      // [E] exclusive end of each expert's rows
  int32_t* tiles;        // [max_tiles][4]: expert, row0, rows, 0
  int32_t* token_map;    // [A]
  int32_t* inverse_map;  // [A]
  float* row_weight;     // [A]
  uint16_t* act;         // [A + T][I]
  float* contrib;        // [A + T][H]
  uint16_t* h;           // [T][H]   (stack only)
  uint16_t* r[2];        // [T][H]   (stack only)
};

struct PrefillDims {
  int64_t T, A, nb, max_tiles;
  int E, k, H, I;
};

static PrefillDims prefill_dims(const aima_moe_layer* L, int64_t T, int k) {
  PrefillDims d;
  d.T = T;
  d.k = k;
  d.A = T * k;
  d.E = L->experts;
  d.H = L->hidden;
  d.I = L->inter;
  d.nb = (d.A + kSchedBlock - 1) / kSchedBlock;
  d.max_tiles = (d.A + kBM - 1) / kBM + std::min<int64_t>(d.E, d.A) + (T + kBM - 1) / kBM;
  return d;
}

enum class WsMode { kSchedule, kLayer, kStack };

// Carves the workspace (base may be null to only measure it); returns bytes.
static size_t prefill_ws_layout(const PrefillDims& d, WsMode mode, void* base, PrefillWs* w) {
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    const size_t at = off;
    off += round_up(bytes, 256);
    return p ? p + at : nullptr;
  };
  PrefillWs l{};
  char* hdr = take(kWsHeader);
  l.err = reinterpret_cast<uint32_t*>(hdr);
  l.tile_count = reinterpret_cast<int32_t*>(hdr ? hdr + 64 : nullptr);
  l.block_base = reinterpret_cast<int32_t*>(take((size_t)d.nb * d.E * 4));
  l.offsets = reinterpret_cast<int32_t*>(take((size_t)d.E * 4));
  l.tiles = reinterpret_cast<int32_t*>(take((size_t)d.max_tiles * 16));
  l.token_map = reinterpret_cast<int32_t*>(take((size_t)d.A * 4));
  l.inverse_map = reinterpret_cast<int32_t*>(take((size_t)d.A * 4));
  l.row_weight = reinterpret_cast<float*>(take((size_t)d.A * 4));
  if (mode != WsMode::kSchedule) {
    l.act = reinterpret_cast<uint16_t*>(take((size_t)(d.A + d.T) * d.I * 2));
    l.contrib = reinterpret_cast<float*>(take((size_t)(d.A + d.T) * d.H * 4));
  }
  if (mode == WsMode::kStack) {
    l.h = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
    l.r[0] = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
    l.r[1] = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
  }
  if (w) *w = l;
  return off;
}

// ---------------------------------------------------------------------------
// schedule
// ---------------------------------------------------------------------------

// Mask of the lanes (among `active`) holding the same expert id; `bits`
// covers the id range.  Eight-or-ten ballots replace a match-any.
__device__ __forceinline__ uint64_t match_mask(int e, uint64_t active, int bits) {
  uint64_t m = active;
  for (int b = 0; b < bits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

// Reads assignment a, validates it (range, duplicate within the token) and
// returns the expert id clamped into range so that every later index stays
// inside its buffer even for invalid input.
__device__ __forceinline__ int sched_expert(const int32_t* __restrict__ ids, int64_t a, int k,
                                            int E, uint32_t* err) {
  const int e = ids[a];
  const int rank = (int)(a % k);
  uint32_t bad = 0;
  if (e < 0 || e >= E) bad |= AIMA_DEVERR_EXPERT_RANGE;
  for (int p = 0; p < rank; ++p) {
    if (ids[a - rank + p] == e) bad |= AIMA_DEVERR_EXPERT_DUPLICATE;
  }
  if (bad) atomicOr(err, bad);
  return (e < 0 || e >= E) ? 0 : e;
}

__global__ __launch_bounds__(64) void sched_count_kernel(const int32_t* __restrict__ ids,
                                                         int64_t A, int k, int E, int bits,
                                                         uint32_t* err,
                                                         int32_t* __restrict__ block_counts) {
  __shared__ int cnt[kMaxExperts];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) cnt[e] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSchedBlock;
  for (int sub = 0; sub < kSchedBlock / 64; ++sub) {
    const int64_t a = base + sub * 64 + lane;
    const bool valid = a < A;
    const int e = valid ? sched_expert(ids, a, k, E, err) : 0;
    const uint64_t act = __ballot(valid);
    if (act == 0) break;
    const uint64_t m = match_mask(e, act, bits);
    if (valid && lane == __ffsll((unsigned long long)m) - 1) cnt[e] += __popcll(m);
    __syncthreads();
  }
  for (int e = lane; e < E; e += 64) block_counts[(int64_t)blockIdx.x * E + e] = cnt[e];
}

// Exclusive scan over the 1024 threads of a block; returns the prefix and
// writes the grand total to *total.
__device__ int block_exclusive_scan_1024(int v, int* smem, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(inc, off, 64);
    if (lane >= off) inc += t;
  }
  if (lane == 63) smem[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < 16; ++w) {
      const int t = smem[w];
      smem[w] = run;
      run += t;
    }
    smem[16] = run;
  }
  __syncthreads();
  const int r = smem[wave] + inc - v;
  *total = smem[16];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(1024) void sched_scan_kernel(int32_t* __restrict__ block_base,
                                                          int64_t nb, int E, int64_t T,
                                                          int64_t A, int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ tiles,
                                                          int32_t* __restrict__ tile_count) {
  __shared__ int smem[32];
  const int e = threadIdx.x;
  int total = 0;
  if (e < E) {
    for (int64_t b = 0; b < nb; ++b) {
      const int c = block_base[b * E + e];
      block_base[b * E + e] = total;
      total += c;
    }
  }
  const int ntiles = (total + kBM - 1) / kBM;
  int all_rows, all_tiles;
  const int begin = block_exclusive_scan_1024(total, smem, &all_rows);
  const int tbegin = block_exclusive_scan_1024(ntiles, smem, &all_tiles);
  if (e < E) {
    for (int64_t b = 0; b < nb; ++b) block_base[b * E + e] += begin;
    offsets[e] = begin + total;
    for (int t = 0; t < ntiles; ++t) {
      int32_t* td = tiles + 4 * (int64_t)(tbegin + t);
      td[0] = e;
      td[1] = begin + t * kBM;
      td[2] = min(kBM, total - t * kBM);
      td[3] = 0;
    }
  }
  const int64_t shared_tiles = (T + kBM - 1) / kBM;
  for (int64_t t = e; t < shared_tiles; t += 1024) {
    int32_t* td = tiles + 4 * (all_tiles + t);
    td[0] = E;
    td[1] = (int)(A + t * kBM);
    td[2] = (int)min((int64_t)kBM, T - t * kBM);
    td[3] = 0;
  }
  if (e == 0) *tile_count = all_tiles + (int)shared_tiles;
}

__global__ __launch_bounds__(64) void sched_scatter_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ weights, int64_t A, int k, int E,
    int bits, const int32_t* __restrict__ block_base, int32_t* __restrict__ token_map,
    int32_t* __restrict__ inverse_map, float* __restrict__ row_weight) {
  __shared__ int cur[kMaxExperts];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) cur[e] = block_base[(int64_t)blockIdx.x * E + e];
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSchedBlock;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int sub = 0; sub < kSchedBlock / 64; ++sub) {
    const int64_t a = base + sub * 64 + lane;
    const bool valid = a < A;
    int e = 0;
    if (valid) {
      const int raw = ids[a];
      e = (raw < 0 || raw >= E) ? 0 : raw;
    }
    const uint64_t act = __ballot(valid);
    if (act == 0) break;
    const uint64_t m = match_mask(e, act, bits);
    const int pos = cur[e] + __popcll(m & below);
    __syncthreads();
    if (valid) {
      token_map[pos] = (int32_t)(a / k);
      inverse_map[a] = pos;
      row_weight[pos] = weights[a];
      if (lane == __ffsll((unsigned long long)m) - 1) cur[e] += __popcll(m);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 permute_pairs(u32x4 v) {
  // (x0,x1)(x2,x3)(x4,x5)(x6,x7) -> (x0,x4)(x1,x5)(x2,x6)(x3,x7)
  return u32x4{__builtin_amdgcn_perm(v[2], v[0], 0x05040100u),
               __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
               __builtin_amdgcn_perm(v[3], v[1], 0x05040100u),
               __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
}

// 8 nibbles (k0..k7) -> exact f16 (q - z) in MFMA slot order k0,k4,k1,k5,k2,k6,k3,k7.
__device__ __forceinline__ f16x8 dequant8(uint32_t d, uint32_t zz) {
  const f16x2 zh = as_h2(zz);
  const f16x2 p0 = as_h2((d & 0x000F000Fu) | 0x64006400u) - zh;
  const f16x2 p1 = as_h2(((d >> 4) & 0x000F000Fu) | 0x64006400u) - zh;
  const f16x2 p2 = as_h2(((d >> 8) & 0x000F000Fu) | 0x64006400u) - zh;
  const f16x2 p3 = as_h2(((d >> 12) & 0x000F000Fu) | 0x64006400u) - zh;
  const u32x4 v{h2_bits(p0), h2_bits(p1), h2_bits(p2), h2_bits(p3)};
  return __builtin_bit_cast(f16x8, v);
}

template <bool GATEUP>
__global__ __launch_bounds__(256, 1) void grouped_gemm_kernel(
    aima_moe_layer L, const uint16_t* __restrict__ src, const int32_t* __restrict__ tiles,
    const int32_t* __restrict__ tile_count, const int32_t* __restrict__ token_map,
    const float* __restrict__ row_weight, int64_t A, uint16_t* __restrict__ act_out,
    float* __restrict__ contrib_out) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kLdsRowHalves];
  const int tile = blockIdx.x;
  if (tile >= *tile_count) return;
  const int e = tiles[4 * tile + 0];
  const int64_t row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  const int E = L.experts;
  const int64_t H = L.hidden, I = L.inter;
  const int64_t K = GATEUP ? H : I;
  const int GK = (int)(K / 128);
  const int64_t rows_e = GATEUP ? 2 * I : H;

  const aima_u4_tensor& W = GATEUP ? (e < E ? L.gate_up : L.shared_gate_up)
                                   : (e < E ? L.down : L.shared_down);
  const int64_t eoff = (e < E) ? e : 0;
  const uint8_t* qw = W.qweight + eoff * rows_e * (K / 2);
  const uint16_t* sc = W.scale + eoff * rows_e * GK;
  const uint8_t* zp = W.zp + eoff * (rows_e * GK / 2);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;

  // B rows owned by this lane (one per N block).
  int64_t wr[2];
  if (GATEUP) {
    const int64_t jb = (int64_t)blockIdx.y * 128 + wave * 32;
    wr[0] = jb + n;
    wr[1] = I + jb + n;
  } else {
    const int64_t hb = (int64_t)blockIdx.y * 256 + wave * 64;
    wr[0] = hb + n;
    wr[1] = hb + 32 + n;
  }

  // A rows loaded by this thread: rr_i = (tid >> 4) + 16 i, part = tid & 15.
  const int part = tid & 15;
  const uint16_t* arow[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int rr = (tid >> 4) + 16 * i;
    if (rr < rows) {
      const int64_t grow = row0 + rr;
      int64_t srow;
      if (GATEUP) {
        srow = (e < E) ? (int64_t)token_map[grow] : grow - A;
      } else {
        srow = grow;
      }
      arow[i] = src + srow * K + part * 8;
    } else {
      arow[i] = nullptr;
    }
  }

  u32x4 areg[8];
  auto load_a = [&](int g) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      areg[i] = arow[i] ? load16(arow[i] + g * 128) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = (tid >> 4) + 16 * i;
      *reinterpret_cast<u32x4*>(&As[buf][rr * kLdsRowHalves + part * 8]) = permute_pairs(areg[i]);
    }
  };
  u32x4 braw[2][2];
  float bs[2];
  uint32_t bzz[2];
  auto load_b = [&](int g, u32x4 (&raw)[2][2], float (&s)[2], uint32_t (&zz)[2]) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const uint8_t* p = qw + wr[nb] * (K / 2) + g * 64 + hh * 32;
      raw[nb][0] = load16_nt(p);
      raw[nb][1] = load16_nt(p + 16);
      const int64_t gi = wr[nb] * GK + g;
      s[nb] = h2f(sc[gi]);
      zz[nb] = (0x6400u | u4_code(zp, gi)) * 0x00010001u;
    }
  };

  const int mb_active = (rows + 31) / 32;
  f32x16 acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f32x16{};
  }

  load_a(0);
  load_b(0, braw, bs, bzz);
  store_a(0);
  __syncthreads();

  for (int g = 0; g < GK; ++g) {
    const int buf = g & 1;
    u32x4 nraw[2][2];
    float ns[2];
    uint32_t nzz[2];
    const bool more = g + 1 < GK;
    if (more) {
      load_a(g + 1);
      load_b(g + 1, nraw, ns, nzz);
    }
    f32x16 accg[4][2];
    const uint16_t* abase = &As[buf][n * kLdsRowHalves + hh * 64];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f16x8 b[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) b[nb] = dequant8(braw[nb][j >> 2][j & 3], bzz[nb]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < mb_active) {
          const f16x8 a = *reinterpret_cast<const f16x8*>(abase + mb * 32 * kLdsRowHalves + j * 8);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            accg[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                a, b[nb], j == 0 ? f32x16{} : accg[mb][nb], 0, 0, 0);
          }
        }
      }
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb < mb_active) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[mb][nb][v] += bs[nb] * accg[mb][nb][v];
        }
      }
    }
    if (more) {
      store_a(buf ^ 1);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        braw[nb][0] = nraw[nb][0];
        braw[nb][1] = nraw[nb][1];
        bs[nb] = ns[nb];
        bzz[nb] = nzz[nb];
      }
    }
    __syncthreads();
  }

  // Epilogue.  32x32 MFMA output: lane holds column n, rows
  // 8*(v/4) + 4*hh + (v%4) of its M block.
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < mb_active) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = mb * 32 + 8 * (v >> 2) + 4 * hh + (v & 3);
        if (r < rows) {
          const int64_t grow = row0 + r;
          if (GATEUP) {
            act_out[grow * I + (wr[0])] = f2h(silu_mul(acc[mb][0][v], acc[mb][1][v]));
          } else {
            const float wt = (e < E) ? row_weight[grow] : 1.0f;
            contrib_out[grow * H + wr[0]] = wt * acc[mb][0][v];
            contrib_out[grow * H + wr[1]] = wt * acc[mb][1][v];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// combine: out[t] = f16(residual[t] + (sum_r contrib[inv[t][r]] + sigma_t * shared[t]))
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_kernel(
    const float* __restrict__ contrib, const int32_t* __restrict__ inverse_map, int k, int64_t A,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate_vec,
    const uint16_t* __restrict__ residual, int64_t H, uint16_t* __restrict__ out) {
  __shared__ float red[4];
  __shared__ int rowsel[16];
  const int64_t t = blockIdx.x;
  float g = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += 256) g += h2f(gate_vec[i]) * h2f(x[t * H + i]);
  g = block_sum_256(g, red);
  const double gd = g;
  const float sigma = (float)(gd >= 0.0 ? 1.0 / (1.0 + exp(-gd)) : exp(gd) / (1.0 + exp(gd)));
  if (threadIdx.x < k) rowsel[threadIdx.x] = inverse_map[t * k + threadIdx.x];
  __syncthreads();
  const float* shared_row = contrib + (A + t) * H;
  for (int64_t h = threadIdx.x * 4; h < H; h += 1024) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r = 0; r < k; ++r) {
      const float4 c = *reinterpret_cast<const float4*>(contrib + (int64_t)rowsel[r] * H + h);
      s.x += c.x;
      s.y += c.y;
      s.z += c.z;
      s.w += c.w;
    }
    const float4 c = *reinterpret_cast<const float4*>(shared_row + h);
    float o[4] = {s.x + c.x * sigma, s.y + c.y * sigma, s.z + c.z * sigma, s.w + c.w * sigma};
    if (residual) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = h2f(residual[t * H + h + j]) + o[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) out[t * H + h + j] = f2h(o[j]);
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
static int expert_bits(int E) {
  int b = 1;
  while ((1 << b) < E) ++b;
  return b;
}

static int launch_schedule(const int32_t* ids, const float* weights, const PrefillDims& d,
                           const PrefillWs& w, hipStream_t st) {
  const int bits = expert_bits(d.E);
  hipLaunchKernelGGL(sched_count_kernel, dim3((unsigned)d.nb), dim3(64), 0, st, ids, d.A, d.k,
                     d.E, bits, w.err, w.block_base);
  int rc = launch_check("grouped schedule count");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL(sched_scan_kernel, dim3(1), dim3(1024), 0, st, w.block_base, d.nb, d.E, d.T,
                     d.A, w.offsets, w.tiles, w.tile_count);
  rc = launch_check("grouped schedule scan");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL(sched_scatter_kernel, dim3((unsigned)d.nb), dim3(64), 0, st, ids, weights,
                     d.A, d.k, d.E, bits, w.block_base, w.token_map, w.inverse_map,
                     w.row_weight);
  return launch_check("grouped schedule scatter");
}

static int prefill_layer(const aima_moe_layer& L, const uint16_t* x, const uint16_t* residual,
                         const int32_t* ids, const float* weights, uint16_t* out,
                         const PrefillDims& d, const PrefillWs& w, hipStream_t st) {
  int rc = launch_schedule(ids, weights, d, w, st);
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL((grouped_gemm_kernel<true>), dim3((unsigned)d.max_tiles, d.I / 128), dim3(256),
                     0, st, L, x, w.tiles, w.tile_count, w.token_map, w.row_weight, d.A, w.act,
                     w.contrib);
  rc = launch_check("grouped gate/up GEMM");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL((grouped_gemm_kernel<false>), dim3((unsigned)d.max_tiles, d.H / 256),
                     dim3(256), 0, st, L, w.act, w.tiles, w.tile_count, w.token_map,
                     w.row_weight, d.A, w.act, w.contrib);
  rc = launch_check("grouped down GEMM");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)d.T), dim3(256), 0, st, w.contrib,
                     w.inverse_map, d.k, d.A, x, L.shared_gate_vec, residual, (int64_t)d.H, out);
  return launch_check("grouped combine");
}

int check_layer_prefill(const aima_moe_layer* L, int k, bool need_norm) {
  AIMA_REQUIRE(L != nullptr, "moe prefill: null layer");
  AIMA_REQUIRE(L->gate_up.qweight && L->gate_up.scale && L->gate_up.zp && L->down.qweight &&
                   L->down.scale && L->down.zp && L->shared_gate_up.qweight &&
                   L->shared_gate_up.scale && L->shared_gate_up.zp && L->shared_down.qweight &&
                   L->shared_down.scale && L->shared_down.zp && L->shared_gate_vec,
               "moe prefill: null tensor pointer");
  AIMA_REQUIRE(!need_norm || L->norm_weight, "moe prefill: null norm weight");
  AIMA_REQUIRE(L->experts > 0 && L->experts <= kMaxExperts, "moe prefill: experts must be in [1, 1024]");
  AIMA_REQUIRE(k > 0 && k <= 16 && k <= L->experts, "moe prefill: k must be in [1, min(16, experts)]");
  if (L->group != 128) return fail(AIMA_E_UNSUPPORTED, "moe prefill: group must be 128");
  if (L->shared_inter != L->inter) {
    return fail(AIMA_E_UNSUPPORTED, "moe prefill: shared_inter must equal inter");
  }
  if (L->hidden % 256 != 0 || L->inter % 128 != 0 || L->hidden <= 0 || L->inter <= 0) {
    return fail(AIMA_E_UNSUPPORTED, "moe prefill: hidden % 256 and inter % 128 must be 0");
  }
  AIMA_REQUIRE(aligned(L->gate_up.qweight, 16) && aligned(L->down.qweight, 16) &&
                   aligned(L->shared_gate_up.qweight, 16) && aligned(L->shared_down.qweight, 16),
               "moe prefill: qweight pointers must be 16-byte aligned");
  return AIMA_OK;
}

int rmsnorm_launch(const uint16_t* x, const float* weight, int64_t rows, int64_t hidden,
                   float eps, uint16_t* out, hipStream_t st);

}  // namespace aima

using namespace aima;

extern "C" int aima_moe_prefill_workspace_size(const aima_moe_layer* layer, int64_t tokens,
                                               int32_t k, size_t* bytes) {
  AIMA_REQUIRE(layer && bytes, "moe_prefill_workspace_size: null pointer");
  AIMA_REQUIRE(tokens > 0 && k > 0, "moe_prefill_workspace_size: tokens and k must be positive");
  *bytes = prefill_ws_layout(prefill_dims(layer, tokens, k), WsMode::kLayer, nullptr, nullptr);
  return AIMA_OK;
}

extern "C" int aima_moe_stack_prefill_workspace_size(const aima_moe_layer* layer,
                                                     int64_t tokens, int32_t k, size_t* bytes) {
  AIMA_REQUIRE(layer && bytes, "moe_stack_prefill_workspace_size: null pointer");
  AIMA_REQUIRE(tokens > 0 && k > 0, "moe_stack_prefill_workspace_size: tokens and k must be positive");
  *bytes = prefill_ws_layout(prefill_dims(layer, tokens, k), WsMode::kStack, nullptr, nullptr);
  return AIMA_OK;
}

extern "C" int aima_moe_grouped_prefill(const aima_moe_layer* layer, const uint16_t* x,
                                        const uint16_t* residual, int64_t tokens,
                                        const int32_t* ids, const float* weights, int32_t k,
                                        uint16_t* out, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  int rc = check_layer_prefill(layer, k, false);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(x && ids && weights && out, "moe_grouped_prefill: null pointer");
  AIMA_REQUIRE(tokens > 0 && tokens <= (1 << 24), "moe_grouped_prefill: tokens must be in [1, 2^24]");
  AIMA_REQUIRE(aligned(x, 16), "moe_grouped_prefill: x must be 16-byte aligned");
  const PrefillDims d = prefill_dims(layer, tokens, k);
  PrefillWs w{};
  const size_t need = prefill_ws_layout(d, WsMode::kLayer, workspace, &w);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "moe_grouped_prefill: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_grouped_prefill: workspace must be 256-byte aligned");
  return prefill_layer(*layer, x, residual, ids, weights, out, d, w, (hipStream_t)stream);
}

extern "C" int aima_moe_stack_prefill(const aima_moe_layer* layers, int32_t n_layers, float eps,
                                      const uint16_t* x_in, int64_t tokens, const int32_t* ids,
                                      const float* weights, int32_t k, uint16_t* out,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  AIMA_REQUIRE(layers && n_layers > 0, "moe_stack_prefill: need at least one layer");
  AIMA_REQUIRE(x_in && ids && weights && out, "moe_stack_prefill: null pointer");
  AIMA_REQUIRE(tokens > 0 && tokens <= (1 << 24), "moe_stack_prefill: tokens must be in [1, 2^24]");
  for (int32_t l = 0; l < n_layers; ++l) {
    int rc = check_layer_prefill(&layers[l], k, true);
    if (rc != AIMA_OK) return rc;
    AIMA_REQUIRE(layers[l].hidden == layers[0].hidden && layers[l].inter == layers[0].inter &&
                     layers[l].experts == layers[0].experts,
                 "moe_stack_prefill: all layers must share hidden, inter and experts");
  }
  const PrefillDims d = prefill_dims(&layers[0], tokens, k);
  PrefillWs w{};
  const size_t need = prefill_ws_layout(d, WsMode::kStack, workspace, &w);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "moe_stack_prefill: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_stack_prefill: workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* r = x_in;
  for (int32_t l = 0; l < n_layers; ++l) {
    const aima_moe_layer& L = layers[l];
    int rc = rmsnorm_launch(r, L.norm_weight, tokens, L.hidden, eps, w.h, st);
    if (rc != AIMA_OK) return rc;
    uint16_t* dst = (l == n_layers - 1) ? out : w.r[l & 1];
    rc = prefill_layer(L, w.h, r, ids + (int64_t)l * d.A, weights + (int64_t)l * d.A, dst, d, w,
                       st);
    if (rc != AIMA_OK) return rc;
    r = dst;
  }
  return AIMA_OK;
}

// Schedule only (the host BuildGroupedSchedule's outputs on the device):
// offsets [E] (exclusive ends), token_map [A], inverse_map [A],
// compact_weights [A] are copied out of the workspace into caller buffers.
extern "C" int aima_grouped_schedule(const int32_t* ids, const float* weights, int64_t tokens,
                                     int32_t k, int32_t experts, int32_t* offsets,
                                     int32_t* token_map, int32_t* inverse_map,
                                     float* compact_weights, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  AIMA_REQUIRE(ids && weights && offsets && token_map && inverse_map && compact_weights,
               "grouped_schedule: null pointer");
  AIMA_REQUIRE(tokens > 0 && tokens <= (1 << 24), "grouped_schedule: tokens must be in [1, 2^24]");
  AIMA_REQUIRE(experts > 0 && experts <= kMaxExperts, "grouped_schedule: experts must be in [1, 1024]");
  AIMA_REQUIRE(k > 0 && k <= 16 && k <= experts, "grouped_schedule: k must be in [1, min(16, experts)]");
  aima_moe_layer shape{};
  shape.experts = experts;
  shape.hidden = 256;
  shape.inter = 128;
  const PrefillDims d = prefill_dims(&shape, tokens, k);
  PrefillWs w{};
  const size_t need = prefill_ws_layout(d, WsMode::kSchedule, workspace, &w);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "grouped_schedule: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "grouped_schedule: workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_schedule(ids, weights, d, w, st);
  if (rc != AIMA_OK) return rc;
  AIMA_HIP(hipMemcpyAsync(offsets, w.offsets, (size_t)experts * 4, hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(token_map, w.token_map, (size_t)d.A * 4, hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(inverse_map, w.inverse_map, (size_t)d.A * 4, hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(compact_weights, w.row_weight, (size_t)d.A * 4, hipMemcpyDeviceToDevice,
                          st));
  return AIMA_OK;
}

extern "C" int aima_grouped_schedule_workspace_size(int64_t tokens, int32_t k, int32_t experts,
                                                    size_t* bytes) {
  AIMA_REQUIRE(bytes && tokens > 0 && k > 0 && experts > 0,
               "grouped_schedule_workspace_size: invalid arguments");
  aima_moe_layer shape{};
  shape.experts = experts;
  shape.hidden = 256;
  shape.inter = 128;
  *bytes = prefill_ws_layout(prefill_dims(&shape, tokens, k), WsMode::kSchedule, nullptr,
                             nullptr);
  return AIMA_OK;
}
