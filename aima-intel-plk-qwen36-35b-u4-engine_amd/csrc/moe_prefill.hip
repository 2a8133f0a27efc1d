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
#pragma unroll
  for (int b = 0; b < 10; ++b) {  // ids < kMaxExperts = 2^10
    if (b < bits) {
      const bool bit = (e >> b) & 1;
      const uint64_t bal = __ballot(bit);
      m &= bit ? bal : ~bal;
    }
  }
  return m;
}

// The block's kSchedBlock ids, staged in LDS with coalesced 16-byte loads
// (the per-assignment work below then never waits on global memory).
__device__ __forceinline__ void stage_ids(const int32_t* __restrict__ ids, int64_t base, int64_t A,
                                          int32_t* sid) {
  const int lane = threadIdx.x;
  if (base + kSchedBlock <= A && (reinterpret_cast<uintptr_t>(ids + base) & 15) == 0) {
#pragma unroll
    for (int i = 0; i < kSchedBlock / 256; ++i) {
      const int q = lane + 64 * i;
      reinterpret_cast<u32x4*>(sid)[q] = *reinterpret_cast<const u32x4*>(ids + base + 4 * q);
    }
  } else {
    for (int i = lane; i < kSchedBlock; i += 64) sid[i] = base + i < A ? ids[base + i] : 0;
  }
  __syncthreads();
}

// Validates assignment a (range, duplicate within its token) from the staged
// ids (earlier ids of a token that starts in the previous block are read from
// global memory) and returns the expert id clamped into range, so every later
// index stays inside its buffer even for invalid input.
__device__ __forceinline__ int sched_expert(const int32_t* __restrict__ ids, const int32_t* sid,
                                            int64_t base, int64_t a, int k, int E, uint32_t* err) {
  const int e = sid[a - base];
  const int rank = (int)(a % k);
  const int64_t t0 = a - rank;  // first assignment of the token
  uint32_t bad = 0;
  if (e < 0 || e >= E) bad |= AIMA_DEVERR_EXPERT_RANGE;
  if (t0 >= base) {
    // all earlier ids of the token are staged: independent, unconditional LDS
    // reads (indices clamped into the block), compared only below `rank`
    const int t0l = (int)(t0 - base);
#pragma unroll
    for (int p = 0; p < 15; ++p) {
      const int o = sid[min(t0l + p, kSchedBlock - 1)];
      if (p < rank && o == e) bad |= AIMA_DEVERR_EXPERT_DUPLICATE;
    }
  } else {
    for (int p = 0; p < rank; ++p) {
      const int64_t b = t0 + p;
      const int o = b >= base ? sid[b - base] : ids[b];
      if (o == e) bad |= AIMA_DEVERR_EXPERT_DUPLICATE;
    }
  }
  if (bad) atomicOr(err, bad);
  return (e < 0 || e >= E) ? 0 : e;
}

__global__ __launch_bounds__(64) void sched_count_kernel(const int32_t* __restrict__ ids,
                                                         int64_t A, int k, int E, int bits,
                                                         uint32_t* err,
                                                         int32_t* __restrict__ block_counts) {
  __shared__ int cnt[kMaxExperts];
  __shared__ __attribute__((aligned(16))) int32_t sid[kSchedBlock];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) cnt[e] = 0;
  const int64_t base = (int64_t)blockIdx.x * kSchedBlock;
  stage_ids(ids, base, A, sid);
  for (int sub = 0; sub < kSchedBlock / 64; ++sub) {
    const int64_t a = base + sub * 64 + lane;
    const bool valid = a < A;
    const int e = valid ? sched_expert(ids, sid, base, a, k, E, err) : 0;
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
    // eight independent loads in flight per step
    for (int64_t b0 = 0; b0 < nb; b0 += 8) {
      int c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = b0 + j < nb ? block_base[(b0 + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (b0 + j < nb) block_base[(b0 + j) * E + e] = total;
        total += c[j];
      }
    }
  }
  const int ntiles = (total + kBM - 1) / kBM;
  int all_rows, all_tiles;
  const int begin = block_exclusive_scan_1024(total, smem, &all_rows);
  const int tbegin = block_exclusive_scan_1024(ntiles, smem, &all_tiles);
  if (e < E) {
    for (int64_t b = 0; b < nb; ++b) block_base[b * E + e] += begin;  // independent stores
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
  __shared__ __attribute__((aligned(16))) int32_t sid[kSchedBlock];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) cur[e] = block_base[(int64_t)blockIdx.x * E + e];
  const int64_t base = (int64_t)blockIdx.x * kSchedBlock;
  stage_ids(ids, base, A, sid);
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // the block's router weights, loaded up front (independent loads)
  float wv[kSchedBlock / 64];
#pragma unroll
  for (int sub = 0; sub < kSchedBlock / 64; ++sub) {
    const int64_t a = base + sub * 64 + lane;
    wv[sub] = a < A ? weights[a] : 0.f;
  }
#pragma unroll
  for (int sub = 0; sub < kSchedBlock / 64; ++sub) {
    const int64_t a = base + sub * 64 + lane;
    const bool valid = a < A;
    int e = 0;
    if (valid) {
      const int raw = sid[a - base];
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
      row_weight[pos] = wv[sub];
      if (lane == __ffsll((unsigned long long)m) - 1) cur[e] += __popcll(m);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
// 8 nibbles k0..k7 of one 32-bit word -> f16 (q - z) * s in natural order
// (k0,k1),(k2,k3),(k4,k5),(k6,k7).  A byte permute copies byte i to bytes 0
// and 2; masking 0x00F0000F leaves the even nibble as 1024 + q (low half) and
// the odd one as 1024 + 16 q (high half), which use zz2 = {1024+z, 1024+16z}
// and ss2 = {s, s/16}.  (q - z) is exact in f16 and (q - z) * s is rounded
// once (relative error <= 2^-11), which keeps the group scale out of the f32
// accumulators.  `magic` is 0x64006400 in a VGPR (one v_and_or_b32 per pair).
__device__ __forceinline__ f16x8 dequant8(uint32_t d, f16x2 zz2, f16x2 ss2, uint32_t magic) {
  const f16x2 p0 = (as_h2((__builtin_amdgcn_perm(d, d, 0x0C000C00u) & 0x00F0000Fu) | magic) - zz2) * ss2;
  const f16x2 p1 = (as_h2((__builtin_amdgcn_perm(d, d, 0x0C010C01u) & 0x00F0000Fu) | magic) - zz2) * ss2;
  const f16x2 p2 = (as_h2((__builtin_amdgcn_perm(d, d, 0x0C020C02u) & 0x00F0000Fu) | magic) - zz2) * ss2;
  const f16x2 p3 = (as_h2((__builtin_amdgcn_perm(d, d, 0x0C030C03u) & 0x00F0000Fu) | magic) - zz2) * ss2;
  const u32x4 v{h2_bits(p0), h2_bits(p1), h2_bits(p2), h2_bits(p3)};
  return __builtin_bit_cast(f16x8, v);
}

// Direct global -> LDS loads (each lane's 16 or 4 bytes land at the
// wave-uniform LDS address + lane * size), addressed as a wave-uniform base
// (SGPRs) plus a 32-bit per-lane byte offset.  Issued through inline
// assembly: the compiler then neither counts them nor orders LDS reads behind
// them; the kernel waits for them itself (s_waitcnt vmcnt before its
// barriers).  The s_nop gives the M0 write one wait state before its use.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ uint32_t lds_addr(const void* lds) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)lds);
}
// `lds` is the wave-uniform LDS byte address (see lds_addr).
__device__ __forceinline__ void lds_load16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}
__device__ __forceinline__ void lds_load4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}

// One block computes a 128-row M tile of one expert against 256 weight rows:
// gate/up: 128 gate + 128 up rows (the same 128 intermediate columns), down:
// 256 output columns.  8 waves; wave w owns all 128 M rows and one 32-column
// block: (gate/up) gate rows j0 + 16 w .. +16 in MFMA columns 0..15 and the
// matching up rows in columns 16..31, (down) rows 32 w .. +32.  So each
// weight element is dequantized by exactly one lane of the block, and a lane
// feeds 4 MFMAs (32x32x16, one per 32-row M block) with every dequantized
// weight.  Two waves per SIMD.  The K loop runs over 128-wide quantization
// groups.
//
// All operands of a group reach LDS by direct global->LDS loads (no register
// staging), three groups in flight: the A tile (128 rows x 256 bytes,
// gathered through the token map; piece p of row r sits in slot p ^ (r & 15)
// so MFMA operand reads are free of bank conflicts), the packed weight bytes
// of the 256 rows (16 KB, in the order the lanes consume them), and each
// row's scale and zero-point words.
//
// Blocks are mapped XCD-aware: physical block p runs on XCD p % 8 (round-robin
// dispatch), and each XCD walks a contiguous range of (M tile, N tile) pairs,
// N tile fastest, so the N tiles of one M tile (same A rows) and consecutive M
// tiles of one expert (same weight rows) share that XCD's L2.
constexpr int kGemmThreads = 512;
constexpr int kStageA = kBM * 256;        // bytes
constexpr int kStageB = 256 * 64;         // bytes
constexpr int kStageSZ = 2 * 256 * 4;     // bytes
constexpr int kLoadsPerStage = 7;         // direct loads per wave per group

template <bool GATEUP>
__global__ __launch_bounds__(kGemmThreads, 1) void grouped_gemm_kernel(
    aima_moe_layer L, const uint16_t* __restrict__ src, const int32_t* __restrict__ tiles,
    const int32_t* __restrict__ tile_count, const int32_t* __restrict__ token_map,
    const float* __restrict__ row_weight, int64_t A, int ntiles_n,
    uint16_t* __restrict__ act_out, float* __restrict__ contrib_out) {
  // LDS: three stages of A tiles, weight bytes and scale / zero-point words,
  // then the router weights of the tile's rows (down epilogue)
  constexpr int kOffB = 3 * kStageA, kOffZ = kOffB + 3 * kStageB, kOffW = kOffZ + 3 * kStageSZ;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kOffW + kBM * 4];
  const int total = *tile_count * ntiles_n;
  const int per_xcd = (total + 7) / 8;
  const int p = blockIdx.x;
  const int logical = (p % 8) * per_xcd + p / 8;
  if (p / 8 >= per_xcd || logical >= total) return;
  const int tile = logical / ntiles_n;
  const int ntile = logical - tile * ntiles_n;

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
  const uint8_t* sc = reinterpret_cast<const uint8_t*>(W.scale + eoff * rows_e * GK);
  const uint8_t* zp = W.zp + eoff * (rows_e * GK / 2);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;

  // weight row of MFMA column n_ of column block w_
  auto wrow = [&](int w_, int n_) -> int64_t {
    if (GATEUP) {
      const int64_t j = (int64_t)ntile * 128 + w_ * 16 + (n_ & 15);
      return n_ < 16 ? j : I + j;
    }
    return (int64_t)ntile * 256 + w_ * 32 + n_;
  };
  const int64_t my_row = wrow(wave, n);

  // --- direct-load sources of this lane: uniform bases + 32-bit offsets ---
  // A: block instruction q = 4 wave + i covers rows 4q .. 4q+3; lane -> row
  // 4q + lane/16, LDS slot lane%16 holding piece (lane%16) ^ (row & 15).
  // Rows past the tile read the tile's first row (valid memory; their
  // results are never stored).  (Byte offsets stay below 2^31: the host
  // limits tokens * hidden.)
  const void* a_base = uniform_ptr(src);
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (4 * wave + i) + (lane >> 4);
    const int64_t grow = row0 + (r < rows ? r : 0);
    int64_t srow;
    if (GATEUP) {
      srow = (e < E) ? (int64_t)token_map[grow] : grow - A;
    } else {
      srow = grow;
    }
    const int piece = (lane & 15) ^ (r & 15);
    aoff[i] = (uint32_t)((srow * K + piece * 8) * 2);
  }
  // B: wave w loads its own column block: 16-byte piece t of the 32 bytes
  // lane (n, hh) consumes (k 64 hh .. +64 of the group)
  const void* b_base = uniform_ptr(qw);
  const uint32_t boff = (uint32_t)(my_row * (K / 2) + hh * 32);
  // scale / zero-point words: wave w loads word set w: scales for w < 4,
  // zero points for w >= 4; lane -> word (w % 4) * 64 + lane of column block
  // idx / 32, column idx % 32
  int64_t sz_row;
  {
    const int idx = (wave & 3) * 64 + lane;
    sz_row = wrow(idx >> 5, idx & 31);
  }
  const bool sz_is_zero = wave >= 4;
  const void* z_base = uniform_ptr(sz_is_zero ? zp : sc);

  // LDS destinations: the LDS base address plus wave-uniform integer offsets
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int g, int st) {
    const uint32_t la = lds0 + (uint32_t)(st * kStageA + wave * 4096);
    const uint32_t lb = lds0 + (uint32_t)(kOffB + st * kStageB + wave * 2048);
    const uint32_t lz = lds0 + (uint32_t)(kOffZ + st * kStageSZ + wave * 256);
#pragma unroll
    for (int i = 0; i < 4; ++i) lds_load16(a_base, aoff[i] + g * 256, la + i * 1024);
#pragma unroll
    for (int t = 0; t < 2; ++t) lds_load16(b_base, boff + g * 64 + t * 16, lb + t * 1024);
    const int64_t gi = sz_row * GK + g;
    const uint32_t zoff = sz_is_zero ? (uint32_t)((gi >> 1) & ~(int64_t)3)
                                     : (uint32_t)((gi * 2) & ~(int64_t)3);
    lds_load4(z_base, zoff, lz);
  };

  // M blocks that hold rows of the tile
  const int mb_active = min(4, (rows + 31) / 32);
  f32x16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x16{};
  const uint32_t magic = u4_magic();

  auto compute = [&](int g, int st) {
    const uint8_t* sA = smem + st * kStageA;
    const uint8_t* sB = smem + kOffB + st * kStageB;
    const uint32_t* sZ = reinterpret_cast<const uint32_t*>(smem + kOffZ + st * kStageSZ);
    const int col = wave * 32 + n;  // word index within a set
    const uint32_t sw = sZ[col];
    const uint32_t zw = sZ[256 + col];
    const int64_t gi = my_row * GK + g;
    const uint32_t sbits = (sw >> ((gi & 1) * 16)) & 0xffffu;
    const uint32_t z = (zw >> ((gi & 7) * 4)) & 0xfu;
    const f16x2 s2 = as_h2(sbits * 0x00010001u);
    const f16x2 ss2 = f16x2{s2.x, (_Float16)(s2.y * (_Float16)0.0625f)};
    const f16x2 zz2 = as_h2((0x6400u | z) | ((0x6400u | (z << 4)) << 16));
    u32x4 braw[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      braw[t] = *reinterpret_cast<const u32x4*>(sB + ((2 * wave + t) * 64 + lane) * 16);
    }
    auto afrag = [&](int mb, int j) {
      const int m = mb * 32 + n;
      const int slot = (hh * 8 + j) ^ (m & 15);
      return *reinterpret_cast<const f16x8*>(sA + m * 256 + slot * 16);
    };
    // All four M blocks run unconditionally (rows past the tile hold valid
    // copies of row 0 and are never stored): straight-line code in which the
    // A fragments of k-step j+1 load and its weights dequantize while the
    // MFMAs of step j run.
    f16x8 af[2][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) af[0][mb] = afrag(mb, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j + 1 < 8) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) af[(j + 1) & 1][mb] = afrag(mb, j + 1);
      }
      const f16x8 b = dequant8(braw[j >> 2][j & 3], zz2, ss2, magic);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j & 1][mb], b, acc[mb], 0, 0, 0);
      }
    }
  };

  // Pipeline: groups g+1 and g+2 load while g computes.  Before computing g
  // a wave waits for its own loads of g (those of g+1, issued later, may stay
  // in flight), then the barrier makes every wave's loads of g visible and
  // guarantees every wave is done with the stage that g+2 reuses.  The
  // barrier is a plain s_barrier between compiler memory barriers: no fence,
  // so it does not wait for the loads in flight.
  auto sync_stage = [&](bool last) {
    if (!last) {
      asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  static_assert(kLoadsPerStage == 7, "the vmcnt(7) above counts one stage's loads");
  issue(0, 0);
  if (GK > 1) issue(1, 1);
  for (int g = 0, st = 0; g < GK; ++g, st = (st == 2 ? 0 : st + 1)) {
    sync_stage(g + 1 >= GK);
    if (g + 2 < GK) issue(g + 2, st == 0 ? 2 : st - 1);
    compute(g, st);
  }

  // Epilogue.  32x32 MFMA output: lane holds column n, rows
  // 8*(v/4) + 4*hh + (v%4) of its M block.  (down: the rows' router weights
  // are staged in LDS first, one load per row)
  float* s_wt = reinterpret_cast<float*>(smem + kOffW);
  if (!GATEUP) {
    if (tid < kBM) s_wt[tid] = (e < E && tid < rows) ? row_weight[row0 + tid] : 1.0f;
    __syncthreads();
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < mb_active) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = mb * 32 + 8 * (v >> 2) + 4 * hh + (v & 3);
        if (GATEUP) {
          // gate in columns 0..15, up in 16..31 of the same lane half
          const float other = __shfl_xor(acc[mb][v], 16, 64);
          if (n < 16 && r < rows) {
            act_out[(row0 + r) * I + my_row] = f2h(silu_mul(acc[mb][v], other));
          }
        } else if (r < rows) {
          contrib_out[(row0 + r) * H + my_row] = s_wt[r] * acc[mb][v];
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
  {
    const int nt = d.I / 128;
    const unsigned grid = (unsigned)round_up(d.max_tiles * nt, 8);
    hipLaunchKernelGGL((grouped_gemm_kernel<true>), dim3(grid), dim3(kGemmThreads), 0, st, L, x,
                       w.tiles, w.tile_count, w.token_map, w.row_weight, d.A, nt, w.act,
                       w.contrib);
  }
  rc = launch_check("grouped gate/up GEMM");
  if (rc != AIMA_OK) return rc;
  {
    const int nt = d.H / 256;
    const unsigned grid = (unsigned)round_up(d.max_tiles * nt, 8);
    hipLaunchKernelGGL((grouped_gemm_kernel<false>), dim3(grid), dim3(kGemmThreads), 0, st, L,
                       w.act, w.tiles, w.tile_count, w.token_map, w.row_weight, d.A, nt, w.act,
                       w.contrib);
  }
  rc = launch_check("grouped down GEMM");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)d.T), dim3(256), 0, st, w.contrib,
                     w.inverse_map, d.k, d.A, x, L.shared_gate_vec, residual, (int64_t)d.H, out);
  return launch_check("grouped combine");
}

// The grouped GEMM addresses its A rows with 32-bit byte offsets.
static bool prefill_offsets_fit(const aima_moe_layer* L, int64_t tokens, int k) {
  const int64_t limit = (int64_t)1 << 30;  // f16 elements (2^31 bytes)
  return tokens * (k + 1) * L->inter < limit && tokens * L->hidden < limit;
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
  AIMA_REQUIRE(prefill_offsets_fit(layer, tokens, k),
               "moe_grouped_prefill: tokens * (k + 1) * inter and tokens * hidden must stay below "
               "2^30 (split the batch)");
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
  AIMA_REQUIRE(prefill_offsets_fit(layers, tokens, k),
               "moe_stack_prefill: tokens * (k + 1) * inter and tokens * hidden must stay below "
               "2^30 (split the batch)");
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
