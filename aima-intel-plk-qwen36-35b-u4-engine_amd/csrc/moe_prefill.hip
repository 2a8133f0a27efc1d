// Grouped MoE prefill on gfx950.
//
// 1. Device schedule (three launches): a stable counting sort of the T*k
//    (token, rank) assignments by expert.  Rows of one expert are ordered by
//    assignment index, the order of the reference's host BuildGroupedSchedule
//    (grouped_s8_u4_prefill_runtime.cpp:231-346), so the schedule is
//    deterministic and bit-comparable with the CPU restatement.  The scan
//    also emits the M tiles (up to 256 rows of one expert; the shared expert
//    covers all T tokens), ordered by height, tallest first.
// 2. Grouped gate/up GEMM (MFMA v_mfma_f32_32x32x16_f16): per tile, the token
//    rows are gathered into LDS; each wave dequantizes its own 32 weight rows
//    straight into MFMA operands as f16 (q - z) * s and multiplies them with
//    every token row of the tile.  The SwiGLU epilogue scales each row by its
//    router weight (1 for the shared expert) and writes f16 [rows][I].
// 3. Grouped down GEMM, same structure over K = I; its output rows are then
//    the weighted contributions, written as f16 [rows][H].
// 4. Combine: per token, the k contributions in rank order, plus the
//    sigmoid-gated shared row, plus the residual, summed in f32 and rounded
//    to f16.
//
// f16 rather than bf16 operands: the activations arrive as f16 and (q - z) is
// an integer in [-15, 15], so (q - z) * s is the only operand rounding (once,
// relative error <= 2^-11) besides the f16 SwiGLU output and the f16
// contributions (the reference's GPU path also keeps f16 contributions,
// grouped_s8_u4_f16_contribution_moe.cl:831-845); MI355X runs dense f16 and
// bf16 MFMA at the same rate.
#include "common.h"

#include <math.h>

#include <algorithm>

namespace aima {

constexpr int kBM = 256;            // rows per M tile (8 MFMA blocks of 32)
constexpr int kSchedBlock = 1024;   // assignments per schedule block
constexpr int kMaxExperts = 1024;
constexpr int kTileClasses = 8;     // tile heights 32, 64, ..., 256 rows

struct PrefillWs {
  uint32_t* err;
  int32_t* tile_count;
  int32_t* block_base;   // [nb][E] block counts, then global row bases
  int32_t* offsets;      // [E] exclusive end of each expert's rows
  int32_t* tiles;        // [max_tiles][4]: expert, row0, rows, 0
  int32_t* token_map;    // [A]
  int32_t* inverse_map;  // [A] (local ranks between count and scatter)
  float* row_weight;     // [A]
  uint16_t* act;         // [A + T][I] f16
  uint16_t* contrib;     // [A + T][H] f16
  uint16_t* x16;         // [T][H] f16 copy of an f32 input (layer calls)
  uint16_t* h;           // [T][H]   (stack only)
  uint16_t* r[2];        // [T][H]   (stack only)
  float* sigma[2];       // [T]      (stack only: shared-expert gates, by layer parity)
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
  // every expert with rows adds at most one partial tile
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
    l.contrib = reinterpret_cast<uint16_t*>(take((size_t)(d.A + d.T) * d.H * 2));
    l.x16 = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
  }
  if (mode == WsMode::kStack) {
    l.h = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
    l.r[0] = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
    l.r[1] = reinterpret_cast<uint16_t*>(take((size_t)d.T * d.H * 2));
    l.sigma[0] = reinterpret_cast<float*>(take((size_t)d.T * 4));
    l.sigma[1] = reinterpret_cast<float*>(take((size_t)d.T * 4));
  }
  if (w) *w = l;
  return off;
}

// ---------------------------------------------------------------------------
// schedule
// ---------------------------------------------------------------------------

// Mask of the lanes (among `active`) holding the same expert id; `bits`
// covers the id range.  Up to ten ballots replace a match-any.
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

// The top-k ids of token t start at ids + t * stride (stride in int32 words,
// >= k): RunLayer's byte topk_stride (grouped_s8_u4_prefill_runtime.hpp:62-84).
__device__ __forceinline__ int32_t topk_id(const int32_t* __restrict__ ids, int32_t a, int k,
                                           int stride) {
  return ids[(int64_t)(a / k) * stride + a % k];
}

// One thread per assignment.  Validates the id (range, duplicate among the
// earlier ranks of its token), ranks it among the block's assignments of the
// same expert in assignment order (ballot match inside each wave plus the
// counts of the earlier waves), and writes the block's per-expert counts.
// The local rank is parked in inverse_map until the scatter.
__global__ __launch_bounds__(kSchedBlock) void sched_count_kernel(
    const int32_t* __restrict__ ids, int stride, int32_t A, int k, int E, int bits, uint32_t* err,
    int32_t* __restrict__ block_counts, int32_t* __restrict__ local_rank) {
  __shared__ int cnt[kSchedBlock / 64][kMaxExperts];
  __shared__ int32_t sid[16 + kSchedBlock];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t base = (int32_t)blockIdx.x * kSchedBlock;
  for (int w = 0; w < kSchedBlock / 64; ++w) {
    for (int e = tid; e < E; e += kSchedBlock) cnt[w][e] = 0;
  }
  // the block's ids and the 16 before them (earlier ranks of a token that
  // starts in the previous block)
  for (int i = tid; i < 16 + kSchedBlock; i += kSchedBlock) {
    const int32_t a = base - 16 + i;
    sid[i] = (a >= 0 && a < A) ? topk_id(ids, a, k, stride) : -1;
  }
  __syncthreads();
  const int32_t a = base + tid;
  const bool valid = a < A;
  int e = 0;
  if (valid) {
    const int raw = sid[16 + tid];
    const int rank = a % k;
    uint32_t bad = (raw < 0 || raw >= E) ? AIMA_DEVERR_EXPERT_RANGE : 0u;
#pragma unroll
    for (int p = 1; p < 16; ++p) {
      if (p <= rank && sid[16 + tid - p] == raw) bad |= AIMA_DEVERR_EXPERT_DUPLICATE;
    }
    if (bad) atomicOr(err, bad);
    e = (raw < 0 || raw >= E) ? 0 : raw;
  }
  const uint64_t m = match_mask(e, __ballot(valid), bits);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int wrank = __popcll(m & below);
  if (valid && wrank == 0) cnt[wave][e] = __popcll(m);
  __syncthreads();
  if (valid) {
    int r = wrank;
    for (int w = 0; w < wave; ++w) r += cnt[w][e];
    local_rank[a] = r;
  }
  for (int x = tid; x < E; x += kSchedBlock) {
    int s = 0;
#pragma unroll
    for (int w = 0; w < kSchedBlock / 64; ++w) s += cnt[w][x];
    block_counts[(int64_t)blockIdx.x * E + x] = s;
  }
}

// Exclusive scans of N values per thread over the 1024 threads of a block
// at once: v[i] becomes the sum of v[i] over the earlier threads, tot[i] the
// sum over all threads.  `smem` holds 17 * N ints.
template <int N>
__device__ void block_exclusive_scan_1024(int (&v)[N], int (&tot)[N], int* smem) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) inc[i] = v[i];
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int t = __shfl_up(inc[i], off, 64);
      if (lane >= off) inc[i] += t;
    }
  }
  if (lane == 63) {
#pragma unroll
    for (int i = 0; i < N; ++i) smem[wave * N + i] = inc[i];
  }
  __syncthreads();
  // lane i of wave 0 turns column i into exclusive wave prefixes + total
  if (threadIdx.x < N) {
    int run = 0;
    for (int w = 0; w < 16; ++w) {
      const int x = smem[w * N + threadIdx.x];
      smem[w * N + threadIdx.x] = run;
      run += x;
    }
    smem[16 * N + threadIdx.x] = run;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    v[i] = smem[wave * N + i] + inc[i] - v[i];
    tot[i] = smem[16 * N + i];
  }
  __syncthreads();
}

// Tiles of one expert with `total` rows in class c (1..8 MFMA blocks of 32
// rows): full 256-row tiles are class 8, the remainder tile is class
// ceil(rem / 32).
__device__ __forceinline__ int tiles_in_class(int total, int c) {
  const int rem = total % kBM;
  const int cls = (rem + 31) / 32;
  return (c == kTileClasses ? total / kBM : 0) + (cls == c ? 1 : 0);
}

// One block of 1024 threads: thread (p, e) with e = tid % Ep (Ep = E rounded
// up to a power of two) scans chunk p of expert e's block counts, the chunk
// partial sums are combined through LDS, and the experts' totals are scanned
// into row offsets and into tile positions per class (class 8 first).
__global__ __launch_bounds__(1024) void sched_scan_kernel(int32_t* __restrict__ block_base,
                                                          int32_t nb, int E, int Ep, int32_t T,
                                                          int32_t A, int with_shared,
                                                          int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ tiles,
                                                          int32_t* __restrict__ tile_count) {
  __shared__ int smem[17 * (1 + kTileClasses)];
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int e = tid % Ep, pidx = tid / Ep, P = 1024 / Ep;
  const int chunk = (nb + P - 1) / P;
  const int b0 = pidx * chunk, b1 = min(nb, b0 + chunk);
  int sum = 0;
  if (e < E) {
    for (int b = b0; b < b1; b += 16) {
      int c[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = b + j < b1 ? block_base[(int64_t)(b + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) sum += c[j];
    }
  }
  part[tid] = sum;
  __syncthreads();
  int before = 0, total = 0;
  for (int q = 0; q < P; ++q) {
    const int v = part[q * Ep + e];
    if (q < pidx) before += v;
    total += v;
  }
  const bool rep = pidx == 0 && e < E;
  // one scan for the row offsets and the tile counts of every class
  // (v[0] rows, v[c] tiles of class c)
  int v[1 + kTileClasses], tot[1 + kTileClasses];
  v[0] = rep ? total : 0;
#pragma unroll
  for (int c = 1; c <= kTileClasses; ++c) v[c] = rep ? tiles_in_class(total, c) : 0;
  block_exclusive_scan_1024<1 + kTileClasses>(v, tot, smem);
  const int begin = v[0];
  if (rep) offsets[e] = begin + total;
  // expert e's row base reaches every chunk thread through LDS
  if (pidx == 0) part[e] = begin;
  __syncthreads();
  if (e < E) {
    int run = part[e] + before;
    for (int b = b0; b < b1; b += 16) {
      int c[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = b + j < b1 ? block_base[(int64_t)(b + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (b + j < b1) block_base[(int64_t)(b + j) * E + e] = run;
        run += c[j];
      }
    }
  }
  // Tiles, by class (tallest first); the shared expert's tiles follow the
  // routed ones of each class.  An expert has full tiles (class 8) and at
  // most one remainder tile of class ceil(rem / 32).
  int cbase[kTileClasses + 1];
  int all_tiles = 0;
#pragma unroll
  for (int c = kTileClasses; c >= 1; --c) {
    cbase[c] = all_tiles;
    all_tiles += tot[c] + (with_shared ? tiles_in_class(T, c) : 0);
  }
  auto place = [&](int ex, int row_begin, int rows_total, int first8, int rem_pos_if_not8) {
    const int full = rows_total / kBM, rem = rows_total % kBM;
    for (int i = 0; i < full; ++i) {
      int32_t* td = tiles + 4 * (int64_t)(first8 + i);
      td[0] = ex;
      td[1] = row_begin + i * kBM;
      td[2] = kBM;
      td[3] = 0;
    }
    if (rem) {
      const int at = (rem + 31) / 32 == kTileClasses ? first8 + full : rem_pos_if_not8;
      int32_t* td = tiles + 4 * (int64_t)at;
      td[0] = ex;
      td[1] = row_begin + full * kBM;
      td[2] = rem;
      td[3] = 0;
    }
  };
  auto rem_slot = [&](int rows_total, const int (&prefix)[1 + kTileClasses]) {
    const int cls = (rows_total % kBM + 31) / 32;
    int pos = 0;
#pragma unroll
    for (int c = 1; c < kTileClasses; ++c) {
      if (c == cls) pos = cbase[c] + prefix[c];
    }
    return pos;
  };
  if (rep) place(e, begin, total, cbase[kTileClasses] + v[kTileClasses], rem_slot(total, v));
  if (tid == 0) {
    if (with_shared) place(E, A, T, cbase[kTileClasses] + tot[kTileClasses], rem_slot(T, tot));
    *tile_count = all_tiles;
  }
}

// One thread per assignment: the row = block base of its expert + its local
// rank.
__global__ __launch_bounds__(kSchedBlock) void sched_scatter_kernel(
    const int32_t* __restrict__ ids, int stride, const float* __restrict__ weights, int32_t A,
    int k, int E, const int32_t* __restrict__ block_base, int32_t* __restrict__ token_map,
    int32_t* __restrict__ inverse_map, float* __restrict__ row_weight) {
  const int32_t a = (int32_t)blockIdx.x * kSchedBlock + threadIdx.x;
  if (a >= A) return;
  const int raw = topk_id(ids, a, k, stride);
  const int e = (raw < 0 || raw >= E) ? 0 : raw;
  const int pos = block_base[(int64_t)blockIdx.x * E + e] + inverse_map[a];
  token_map[pos] = a / k;
  inverse_map[a] = pos;
  row_weight[pos] = weights[a];
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
// The weights enter the MFMAs as f16 (q - z) * s (dequant8, common.h): (q - z)
// is exact in f16 and the product is rounded once (relative error <= 2^-11),
// which keeps the group scale out of the f32 accumulators.

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
// Block barrier that does not wait for outstanding memory operations (the
// waves wait for their own loads first).
__device__ __forceinline__ void plain_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One block computes an M tile (up to 256 token rows of one expert) against
// 256 weight rows: gate/up: 128 gate + 128 up rows (the same 128
// intermediate columns), down: 256 output columns.  8 waves; wave w owns 32
// weight rows and every token row of the tile.  The weights are the MFMA A
// operand (lane l dequantizes weight row l % 32, 8 k values per k-step) and
// the token rows the B operand (MFMA block mb = token rows 32 mb .. +32), so
// each dequantized weight feeds MB MFMAs.  The 32x32 result leaves lane
// (n, hh) with 4 consecutive weight rows 8 q + 4 hh .. +3 (q = 0..3) of token
// row n.  For gate/up the 32 weight rows of a wave are arranged so that
// q = 0, 1 are gate rows and q = 2, 3 the up rows of the same 16 columns;
// SwiGLU needs no lane exchange.
//
// The K loop runs over the 128-wide quantization groups.  Each lane loads
// the packed bytes, scale and zero point of its own weight row straight into
// registers one group ahead.  The token rows of a group (256 rows x 256
// bytes, gathered through the token map) reach LDS by direct global->LDS
// loads into a two-buffer ring; 16-byte piece p of row r sits in slot
// p ^ (r & 15), which keeps the MFMA operand reads free of bank conflicts.
// MB (1..8) is the tile height in 32-row blocks: rows past the tile are
// neither loaded (beyond the MB blocks) nor multiplied.  The epilogue stages
// the output tile in LDS and writes whole rows with 16-byte stores.
//
// Blocks are mapped XCD-aware: physical block p runs on XCD p % 8
// (round-robin dispatch); M tile i goes to XCD i % 8 and the N tiles of one M
// tile (same token rows) are consecutive on that XCD, so they share its L2.
// Tiles come tallest first, so each XCD works through large tiles first.
constexpr int kGemmThreads = 512;
constexpr int kStageA = kBM * 128 * 2;   // token rows of one group, bytes
constexpr int kSmemBytes = 2 * kStageA;  // two-buffer ring; the epilogue reuses it
constexpr int kSmemWeights = kSmemBytes;  // down: router weights of the tile rows (1 KB)

struct GemmTile {
  const void* a_base;     // token rows (uniform)
  const uint8_t* wq;      // this lane's packed weight row (+ its k half)
  const uint16_t* ws;     // this lane's scale row
  const uint8_t* wz;      // packed zero points of the expert
  uint32_t aoff[8];       // per-lane byte offsets of the token-row pieces
  int64_t zbase;          // this lane's zero-point index (row * GK)
  int GK;                 // quantization groups along K
  int e, E, rows;
  int64_t row0;
  int ntile;
};

// silu(g) * u with the hardware exp and reciprocal (relative error ~1e-7;
// exp(-g) = inf for very negative g gives 0, as it should).
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// Optional f32 copies of the GEMM outputs (RunLayer's grouped_swiglu_f32 /
// grouped_contributions_f32, grouped_s8_u4_prefill_runtime.hpp:101-107): the
// SwiGLU rows and the weighted down rows before their f16 rounding, in
// schedule order (null: not written).
struct GemmCapture {
  float* act32;      // [rows][I]
  float* contrib32;  // [rows][H]
};

template <bool GATEUP, int MB>
__device__ __forceinline__ void gemm_tile(const GemmTile& t, uint8_t* smem,
                                          const aima_moe_layer& L,
                                          const float* __restrict__ row_weight,
                                          uint16_t* __restrict__ act_out,
                                          uint16_t* __restrict__ contrib_out,
                                          const GemmCapture& cap) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const uint32_t lds0 = lds_addr(smem);

  // token rows of group g into buffer st: wave w issues block instructions
  // q = w + 8 i (rows 4 q .. 4 q + 3), i < MB
  auto issue = [&](int g, int st) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      lds_load16(t.a_base, t.aoff[i] + g * 256,
                 lds0 + (uint32_t)(st * kStageA + (wave + 8 * i) * 1024));
    }
  };
  struct WGroup {
    u32x4 q0, q1;    // 64 nibbles: k 64 hh .. +64 of the group
    uint32_t s, z;   // f16 scale bits, zero-point byte
  };
  // Global loads by address space: the gate/up row pointers are picked per
  // lane (gate or up tensor), through which the compiler loses the address
  // space (flat loads would also count against the LDS counter).
  auto load_w = [&](int g) {
    WGroup r;
    r.q0 = gload16(t.wq + g * 64);
    r.q1 = gload16(t.wq + g * 64 + 16);
    r.s = ((const AIMA_GLOBAL uint16_t*)t.ws)[g];
    r.z = ((const AIMA_GLOBAL uint8_t*)t.wz)[(t.zbase + g) >> 1];
    return r;
  };

  f32x16 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};
  const uint32_t magic = u4_magic();

  // down: the tile rows' router weights go to LDS with the first loads
  // (waves 0-3, one row per lane; rows past the tile read the first row)
  const bool routed = t.e < t.E;
  if (!GATEUP && routed && wave < kBM / 64) {
    const int r = wave * 64 + lane;
    lds_load4(uniform_ptr(row_weight), (uint32_t)((t.row0 + (r < t.rows ? r : 0)) * 4),
              lds0 + (uint32_t)(kSmemWeights + wave * 256));
  }

  // sA: the group's token rows in LDS, row m at sA + 256 m
  auto compute = [&](int g, const uint8_t* sA, const WGroup& w) {
    const uint32_t z = (w.z >> (((t.zbase + g) & 1) * 4)) & 0xfu;
    const f16x2 ss2 = u4_ss2(w.s);
    const f16x2 zz2 = u4_zz2(z);
    auto bfrag = [&](int mb, int j) {
      const int m = mb * 32 + n;
      const int slot = (hh * 8 + j) ^ (m & 15);
      return *reinterpret_cast<const f16x8*>(sA + m * 256 + slot * 16);
    };
    auto wword = [&](int j) { return j < 4 ? w.q0[j & 3] : w.q1[j & 3]; };
    // Software pipeline over the 8 k-steps: step j issues the operand reads
    // and the dequantization of step j+1, then its MB independent MFMAs (one
    // per accumulator).  The scheduling fences keep each step's MFMAs
    // together: left alone, the scheduler runs all k-steps of one accumulator
    // back to back, and each MFMA then waits for the previous one's result.
    f16x8 bf[2][MB];
    f16x8 a[2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) bf[0][mb] = bfrag(mb, 0);
    a[0] = dequant8(wword(0), zz2, ss2, magic);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j + 1 < 8) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) bf[(j + 1) & 1][mb] = bfrag(mb, j + 1);
        a[(j + 1) & 1] = dequant8(wword(j + 1), zz2, ss2, magic);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j & 1], bf[j & 1][mb], acc[mb], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };


  const int GK = t.GK;
  constexpr int kResidentGroupBytes = MB * 32 * 256;  // token rows of one group
  if (GK * kResidentGroupBytes <= kSmemBytes) {
    // The tile's token rows for the whole K fit in LDS: load them once, one
    // barrier, then every group runs without block synchronization (the
    // waves drift apart, which overlaps one wave's dequantization with
    // another's MFMAs).  Weights stream into registers two groups ahead.
    for (int g = 0; g < GK; ++g) {
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        lds_load16(t.a_base, t.aoff[i] + g * 256,
                   lds0 + (uint32_t)(g * kResidentGroupBytes + (wave + 8 * i) * 1024));
      }
    }
    WGroup w0 = load_w(0);
    WGroup w1 = GK > 1 ? load_w(1) : w0;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    plain_barrier();
    for (int g = 0; g < GK; ++g) {
      const WGroup w = w0;
      w0 = w1;
      if (g + 2 < GK) w1 = load_w(g + 2);
      compute(g, smem + g * kResidentGroupBytes, w);
    }
  } else {
    // Pipeline: group g+1 loads (token rows into the other buffer, weights
    // into registers) while g computes.  Each iteration first waits for all
    // of this wave's loads (those of g), then the barrier makes every wave's
    // token rows of g visible and guarantees every wave is done with the
    // buffer that g+1 refills.  The barrier itself does not wait for memory.
    issue(0, 0);
    WGroup wn = load_w(0);
    for (int g = 0; g < GK; ++g) {
      const int st = g & 1;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      plain_barrier();
      const WGroup w = wn;
      if (g + 1 < GK) {
        issue(g + 1, st ^ 1);
        wn = load_w(g + 1);
      }
      compute(g, smem + st * kStageA, w);
    }
  }

  // Epilogue: lane (n, hh) of MFMA block mb holds token row m = 32 mb + n and
  // weight rows 8 q + 4 hh + c in acc[mb][4 q + c].  Each lane writes its
  // 8-byte runs into an LDS copy of the output tile (16-byte chunk j of row m
  // at chunk slot j ^ (m % chunks)), then whole rows go out as 16-byte stores.
  const int64_t H = L.hidden, I = L.inter;
  constexpr int kChunks = GATEUP ? 16 : 32;   // 16-byte chunks per tile row
  constexpr int kRowBytes = kChunks * 16;
  // The reference's order (grouped_s8_u4_f16_contribution_moe.cl:627-683):
  // gate/up stores the SwiGLU rows unweighted; down multiplies its output by
  // the row's router weight (shared-expert rows: 1; the combine applies the
  // sigmoid gate).  Lane (n, hh) of block mb owns columns
  // 8 (wave * Q + q) + 4 hh .. +3 of token row m = 32 mb + n.
  float wt[MB];
  const float* s_wt = reinterpret_cast<const float*>(smem + kSmemWeights);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) wt[mb] = (!GATEUP && routed) ? s_wt[mb * 32 + n] : 1.0f;
  __syncthreads();  // every wave is done with the token-row buffers
  const int64_t col_base = (int64_t)t.ntile * (GATEUP ? 128 : 256) + hh * 4;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 32 + n;
    uint8_t* rowp = smem + m * kRowBytes;
    if (GATEUP) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float a[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) a[c] = silu_mul_fast(acc[mb][4 * q + c], acc[mb][8 + 4 * q + c]);
        u32x2 v;
        v.x = pack_h2(a[0], a[1]);
        v.y = pack_h2(a[2], a[3]);
        const int chunk = (wave * 2 + q) ^ (m & (kChunks - 1));
        *reinterpret_cast<u32x2*>(rowp + chunk * 16 + hh * 8) = v;
        if (cap.act32 && m < t.rows) {
          *reinterpret_cast<float4*>(cap.act32 + (t.row0 + m) * I + col_base + (wave * 2 + q) * 8) =
              make_float4(a[0], a[1], a[2], a[3]);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = wt[mb] * acc[mb][4 * q + c];
        u32x2 v;
        v.x = pack_h2(o[0], o[1]);
        v.y = pack_h2(o[2], o[3]);
        const int chunk = (wave * 4 + q) ^ (m & (kChunks - 1));
        *reinterpret_cast<u32x2*>(rowp + chunk * 16 + hh * 8) = v;
        if (cap.contrib32 && m < t.rows) {
          *reinterpret_cast<float4*>(cap.contrib32 + (t.row0 + m) * H + col_base + (wave * 4 + q) * 8) =
              make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
  __syncthreads();
  {
    const int c = tid % kChunks;
    constexpr int kRowsPerPass = kGemmThreads / kChunks;
    uint16_t* out = GATEUP ? act_out : contrib_out;
    const int64_t ld = GATEUP ? I : H;
    const int64_t col0 = (int64_t)t.ntile * (GATEUP ? 128 : 256) + c * 8;
#pragma unroll
    for (int i = 0; i < MB * 32 / kRowsPerPass; ++i) {
      const int m = tid / kChunks + kRowsPerPass * i;
      if (m < t.rows) {
        const u32x4 v =
            *reinterpret_cast<const u32x4*>(smem + m * kRowBytes + ((c ^ (m & (kChunks - 1))) * 16));
        if (GATEUP) {
          *reinterpret_cast<u32x4*>(out + (t.row0 + m) * ld + col0) = v;
        } else {
          // contribution rows are read once, by the combine: nontemporal
          // (-20 us per T=16384 layer; the weights, reused by every M tile
          // of their expert, lose 40-60 us with nontemporal loads)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out + (t.row0 + m) * ld + col0));
        }
      }
    }
  }
}

template <bool GATEUP>
__global__ __launch_bounds__(kGemmThreads, 1) void grouped_gemm_kernel(
    aima_moe_layer L, const uint16_t* __restrict__ src, const int32_t* __restrict__ tiles,
    const int32_t* __restrict__ tile_count, const int32_t* __restrict__ token_map,
    const float* __restrict__ row_weight, int64_t A, int ntiles_n,
    uint16_t* __restrict__ act_out, uint16_t* __restrict__ contrib_out, GemmCapture cap) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes + kBM * 4];
  const int p = blockIdx.x;
  const int slot = p >> 3;
  const int mt = (slot / ntiles_n) * 8 + (p & 7);
  if (mt >= *tile_count) return;

  GemmTile t;
  t.ntile = slot % ntiles_n;
  t.e = tiles[4 * mt + 0];
  t.row0 = tiles[4 * mt + 1];
  t.rows = tiles[4 * mt + 2];
  t.E = L.experts;
  const int64_t H = L.hidden, I = L.inter;
  const int64_t K = GATEUP ? H : I;
  t.GK = (int)(K / 128);

  const bool routed_tile = t.e < t.E;
  const int64_t eoff = routed_tile ? t.e : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // weight row (within the expert) of MFMA row i = lane % 32 of this wave
  // (gate/up: MFMA rows i / 8 = 0, 1 are gate rows, 2, 3 up rows of the same
  // 16 intermediate units; either boundary form of the gate/up tensors)
  int64_t wrow;
  const uint8_t* wq;
  const uint16_t* ws;
  const uint8_t* wz;
  {
    const int i = lane & 31;
    if (GATEUP) {
      const GateUpView V = routed_tile ? routed_gate_up(L) : shared_gate_up(L);
      const int q = i >> 3;
      const int h = q >> 1;
      const int64_t j = (int64_t)t.ntile * 128 + wave * 16 + 8 * (q & 1) + (i & 7);
      wrow = V.row(eoff, h, j);
      // selects, not V.q[h]: indexing the view with a per-lane h puts it in
      // scratch memory, and every tile's first weight loads then wait for a
      // scratch store and load
      wq = h ? V.q[1] : V.q[0];
      ws = h ? V.s[1] : V.s[0];
      wz = h ? V.z[1] : V.z[0];
    } else {
      const aima_u4_tensor& W = routed_tile ? L.down : L.shared_down;
      wrow = eoff * H + (int64_t)t.ntile * 256 + wave * 32 + i;
      wq = W.qweight;
      ws = W.scale;
      wz = W.zp;
    }
  }
  t.wq = wq + wrow * (K / 2) + (lane >> 5) * 32;
  t.ws = ws + wrow * t.GK;
  t.wz = wz;
  t.zbase = wrow * t.GK;

  // Token-row loads: block instruction q covers rows 4 q .. 4 q + 3; lane ->
  // row 4 q + lane / 16, LDS slot lane % 16 holding piece
  // (lane % 16) ^ (row & 15).  Wave w issues q = w + 8 i.  Rows past the tile
  // read the tile's first row (valid memory; their results are never
  // stored).  (Byte offsets stay below 2^31: the host limits tokens * hidden
  // and tokens * (k + 1) * inter.)
  t.a_base = uniform_ptr(src);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * (wave + 8 * i) + (lane >> 4);
    const int64_t grow = t.row0 + (r < t.rows ? r : 0);
    const int64_t srow = GATEUP ? ((t.e < t.E) ? (int64_t)token_map[grow] : grow - A) : grow;
    const int piece = (lane & 15) ^ (r & 15);
    t.aoff[i] = (uint32_t)((srow * K + piece * 8) * 2);
  }

  switch ((t.rows + 31) >> 5) {
    case 1: gemm_tile<GATEUP, 1>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    case 2: gemm_tile<GATEUP, 2>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    case 3: gemm_tile<GATEUP, 3>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    case 4: gemm_tile<GATEUP, 4>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    case 5: gemm_tile<GATEUP, 5>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    case 6: gemm_tile<GATEUP, 6>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    case 7: gemm_tile<GATEUP, 7>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
    default: gemm_tile<GATEUP, 8>(t, smem, L, row_weight, act_out, contrib_out, cap); break;
  }
}

// ---------------------------------------------------------------------------
// combine: out[t] = f16(residual[t] + (sum_r contrib[inv[t][r]] + sigma_t * shared[t]))
// ---------------------------------------------------------------------------
// sigma_t = sigmoid(gate_vec . x[t]) in f64, the dot in row_dot_f16's
// order for every caller (so a precomputed value is bit-identical).
__device__ __forceinline__ float shared_gate_sigma(const uint16_t* __restrict__ gate_vec,
                                                   const uint16_t* __restrict__ xr, int64_t H,
                                                   float* red) {
  const double gd = row_dot_f16(gate_vec, xr, H, red);
  return (float)(gd >= 0.0 ? 1.0 / (1.0 + exp(-gd)) : exp(gd) / (1.0 + exp(gd)));
}

// Layer stacks also fuse the next layer's input: with next_norm set, the
// block RMS-normalizes the row it just wrote (rmsnorm_row, the rmsnorm
// kernel's arithmetic and summation order) into next_h, and computes that layer's
// shared-expert gate into next_sigma, which the next combine reads as
// sigma_in instead of re-reading its input.
struct CombineNext {
  const float* norm;          // next layer's RMSNorm weight (null: no fusion)
  const uint16_t* gate_vec;   // next layer's shared gate vector
  float eps;
  uint16_t* h;                // [T][H] next layer's normalized input
  float* sigma;               // [T]
};

__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t* __restrict__ contrib, const int32_t* __restrict__ inverse_map, int k,
    int64_t A, const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate_vec,
    const float* __restrict__ sigma_in, const uint16_t* __restrict__ residual, int64_t H,
    uint16_t* __restrict__ out, CombineNext next) {
  __shared__ float red[4];
  __shared__ int rowsel[16];
  const int64_t t = blockIdx.x;
  const float sigma = sigma_in ? sigma_in[t] : shared_gate_sigma(gate_vec, x + t * H, H, red);
  if (threadIdx.x < k) rowsel[threadIdx.x] = inverse_map[t * k + threadIdx.x];
  __syncthreads();
  const uint16_t* shared_row = contrib + (A + t) * H;
  for (int64_t h = threadIdx.x * 8; h < H; h += 2048) {
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < k; ++r) {
      const u32x4 c = *reinterpret_cast<const u32x4*>(contrib + (int64_t)rowsel[r] * H + h);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wj = c[j];
        s[2 * j] += h2f((uint16_t)(wj & 0xffffu));
        s[2 * j + 1] += h2f((uint16_t)(wj >> 16));
      }
    }
    const u32x4 c = *reinterpret_cast<const u32x4*>(shared_row + h);
    float o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t wj = c[j];
      o[2 * j] = fmaf(h2f((uint16_t)(wj & 0xffffu)), sigma, s[2 * j]);
      o[2 * j + 1] = fmaf(h2f((uint16_t)(wj >> 16)), sigma, s[2 * j + 1]);
    }
    if (residual) {
      const u32x4 rv = *reinterpret_cast<const u32x4*>(residual + t * H + h);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wj = rv[j];
        o[2 * j] = h2f((uint16_t)(wj & 0xffffu)) + o[2 * j];
        o[2 * j + 1] = h2f((uint16_t)(wj >> 16)) + o[2 * j + 1];
      }
    }
    u32x4 ov;
#pragma unroll
    for (int j = 0; j < 4; ++j) ov[j] = pack_h2(o[2 * j], o[2 * j + 1]);
    *reinterpret_cast<u32x4*>(out + t * H + h) = ov;
  }
  if (next.norm) {
    __syncthreads();  // the row is complete (rmsnorm_row reads it back)
    rmsnorm_row(out + t * H, next.norm, H, next.eps, next.h + t * H, red);
    __syncthreads();
    const float sn = shared_gate_sigma(next.gate_vec, next.h + t * H, H, red);
    if (threadIdx.x == 0) next.sigma[t] = sn;
  }
}

// combine_kernel for H = 2048 and k <= 8 (one 16-byte chunk per thread):
// every load is issued before any use, the rank order comes from the
// inverse map read directly (uniform), and the fused next-layer RMSNorm and
// gate work from the registers just written.  Arithmetic and summation
// order are those of combine_kernel + rmsnorm_row + row_dot_f16, so the two
// kernels agree bit for bit.
__global__ __launch_bounds__(256) void combine2048_kernel(
    const uint16_t* __restrict__ contrib, const int32_t* __restrict__ inverse_map, int k,
    int64_t A, const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate_vec,
    const float* __restrict__ sigma_in, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out, CombineNext next) {
  constexpr int64_t H = 2048;
  constexpr int kMaxK = 8;
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const int h = threadIdx.x * 8;
  u32x4 cr[kMaxK];
#pragma unroll
  for (int r = 0; r < kMaxK; ++r) {
    const int64_t row = inverse_map[t * k + (r < k ? r : k - 1)];
    cr[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(contrib + row * H + h));
  }
  // (each contribution row is read once: nontemporal loads measured -40 us
  // per T=16384 layer)
  const u32x4 cs =
      __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(contrib + (A + t) * H + h));
  const u32x4 rv =
      residual ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(residual + t * H + h))
               : u32x4{0u, 0u, 0u, 0u};
  u32x4 nw0{}, nw1{}, ng{};
  if (next.norm) {
    nw0 = *reinterpret_cast<const u32x4*>(next.norm + h);
    nw1 = *reinterpret_cast<const u32x4*>(next.norm + h + 4);
    ng = *reinterpret_cast<const u32x4*>(next.gate_vec + h);
  }
  const float sigma = sigma_in ? sigma_in[t] : shared_gate_sigma(gate_vec, x + t * H, H, red);
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < kMaxK; ++r) {
    if (r < k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wj = cr[r][j];
        s[2 * j] += h2f((uint16_t)(wj & 0xffffu));
        s[2 * j + 1] += h2f((uint16_t)(wj >> 16));
      }
    }
  }
  float o[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t wj = cs[j];
    o[2 * j] = fmaf(h2f((uint16_t)(wj & 0xffffu)), sigma, s[2 * j]);
    o[2 * j + 1] = fmaf(h2f((uint16_t)(wj >> 16)), sigma, s[2 * j + 1]);
  }
  if (residual) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t wj = rv[j];
      o[2 * j] = h2f((uint16_t)(wj & 0xffffu)) + o[2 * j];
      o[2 * j + 1] = h2f((uint16_t)(wj >> 16)) + o[2 * j + 1];
    }
  }
  u32x4 ov;
#pragma unroll
  for (int j = 0; j < 4; ++j) ov[j] = pack_h2(o[2 * j], o[2 * j + 1]);
  __builtin_nontemporal_store(ov, reinterpret_cast<u32x4*>(out + t * H + h));
  if (next.norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = h2f((uint16_t)(ov[j] & 0xffffu)), hi = h2f((uint16_t)(ov[j] >> 16));
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
    ss = block_sum_256(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)H + next.eps);
    const float wv[8] = {as_f32(nw0[0]), as_f32(nw0[1]), as_f32(nw0[2]), as_f32(nw0[3]),
                         as_f32(nw1[0]), as_f32(nw1[1]), as_f32(nw1[2]), as_f32(nw1[3])};
    u32x4 hv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = h2f((uint16_t)(ov[j] & 0xffffu)) * scale * wv[2 * j];
      const float hi = h2f((uint16_t)(ov[j] >> 16)) * scale * wv[2 * j + 1];
      hv[j] = pack_h2(lo, hi);
    }
    *reinterpret_cast<u32x4*>(next.h + t * H + h) = hv;
    float g = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      g = fmaf(h2f((uint16_t)(ng[j] & 0xffffu)), h2f((uint16_t)(hv[j] & 0xffffu)), g);
      g = fmaf(h2f((uint16_t)(ng[j] >> 16)), h2f((uint16_t)(hv[j] >> 16)), g);
    }
    const double gd = block_sum_256(g, red);
    if (threadIdx.x == 0) {
      next.sigma[t] = (float)(gd >= 0.0 ? 1.0 / (1.0 + exp(-gd)) : exp(gd) / (1.0 + exp(gd)));
    }
  }
}


// RunLayer's output (grouped_s8_u4_prefill_runtime.hpp:100-121): the f32 routed
// sum out[t][h] = sum over ranks r (in order, from 0) of the f16 contribution
// rows, as the reference's iq36_scatter_f16_contributions
// (grouped_s8_u4_f16_contribution_moe.cl:831-845).  One block per token.
__global__ __launch_bounds__(256) void combine_routed_f32_kernel(
    const uint16_t* __restrict__ contrib, const int32_t* __restrict__ inverse_map, int k,
    int64_t H, float* __restrict__ out) {
  __shared__ int rowsel[16];
  const int64_t t = blockIdx.x;
  if (threadIdx.x < k) rowsel[threadIdx.x] = inverse_map[t * k + threadIdx.x];
  __syncthreads();
  for (int64_t h = threadIdx.x * 8; h < H; h += 2048) {
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < k; ++r) {
      const u32x4 c = *reinterpret_cast<const u32x4*>(contrib + (int64_t)rowsel[r] * H + h);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wj = c[j];
        s[2 * j] += h2f((uint16_t)(wj & 0xffffu));
        s[2 * j + 1] += h2f((uint16_t)(wj >> 16));
      }
    }
    float4* o = reinterpret_cast<float4*>(out + t * H + h);
    o[0] = make_float4(s[0], s[1], s[2], s[3]);
    o[1] = make_float4(s[4], s[5], s[6], s[7]);
  }
}

// f32 hidden states (RunLayer's input type) -> f16 GEMM operands, round to
// nearest even; 8 values per thread.
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float4* __restrict__ in,
                                                         int64_t n8, u32x4* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const float4 a = in[2 * i], b = in[2 * i + 1];
  out[i] = u32x4{pack_h2(a.x, a.y), pack_h2(a.z, a.w), pack_h2(b.x, b.y), pack_h2(b.z, b.w)};
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
static int expert_bits(int E) {
  int b = 1;
  while ((1 << b) < E) ++b;
  return b;
}

// stride: int32 words between two tokens' top-k rows; with_shared: emit the
// shared expert's tiles (rows A .. A + T - 1).
static int launch_schedule(const int32_t* ids, int stride, const float* weights,
                           const PrefillDims& d, const PrefillWs& w, bool with_shared,
                           hipStream_t st) {
  const int bits = expert_bits(d.E);
  int Ep = 1;
  while (Ep < d.E) Ep <<= 1;
  hipLaunchKernelGGL(sched_count_kernel, dim3((unsigned)d.nb), dim3(kSchedBlock), 0, st, ids,
                     stride, (int32_t)d.A, d.k, d.E, bits, w.err, w.block_base, w.inverse_map);
  int rc = launch_check("grouped schedule count");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL(sched_scan_kernel, dim3(1), dim3(1024), 0, st, w.block_base, (int32_t)d.nb,
                     d.E, Ep, (int32_t)d.T, (int32_t)d.A, with_shared ? 1 : 0, w.offsets, w.tiles,
                     w.tile_count);
  rc = launch_check("grouped schedule scan");
  if (rc != AIMA_OK) return rc;
  hipLaunchKernelGGL(sched_scatter_kernel, dim3((unsigned)d.nb), dim3(kSchedBlock), 0, st, ids,
                     stride, weights, (int32_t)d.A, d.k, d.E, w.block_base, w.token_map,
                     w.inverse_map, w.row_weight);
  return launch_check("grouped schedule scatter");
}

// How one layer call runs beyond the default (f16 in, routed + shared +
// residual f16 out, dense top-k rows).
struct LayerCall {
  int stride = 0;               // int32 words between top-k rows (0: k)
  bool routed_f32 = false;      // RunLayer output: f32 routed sum, no shared expert
  hipEvent_t ev[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  GemmCapture cap{nullptr, nullptr};  // optional f32 intermediates
};

static int record(hipEvent_t e, hipStream_t st) {
  return e ? hip_check(hipEventRecord(e, st), "hipEventRecord(prefill stage)") : AIMA_OK;
}

// sigma_in: the shared-expert gate per token if already known (null: the
// combine computes it from x); next: fusion of the next layer's input.
static int prefill_layer(const aima_moe_layer& L, const uint16_t* x, const uint16_t* residual,
                         const int32_t* ids, const float* weights, void* out,
                         const PrefillDims& d, const PrefillWs& w, hipStream_t st,
                         const float* sigma_in = nullptr, CombineNext next = CombineNext{},
                         const LayerCall& call = LayerCall{}) {
  int rc = record(call.ev[0], st);
  if (rc != AIMA_OK) return rc;
  rc = launch_schedule(ids, call.stride ? call.stride : d.k, weights, d, w, !call.routed_f32, st);
  if (rc != AIMA_OK) return rc;
  if ((rc = record(call.ev[1], st)) != AIMA_OK) return rc;
  const unsigned mtiles = (unsigned)round_up(d.max_tiles, 8);
  {
    const int nt = d.I / 128;
    hipLaunchKernelGGL((grouped_gemm_kernel<true>), dim3(mtiles * nt), dim3(kGemmThreads), 0, st,
                       L, x, w.tiles, w.tile_count, w.token_map, w.row_weight, d.A, nt, w.act,
                       w.contrib, call.cap);
  }
  rc = launch_check("grouped gate/up GEMM");
  if (rc != AIMA_OK) return rc;
  if ((rc = record(call.ev[2], st)) != AIMA_OK) return rc;
  {
    const int nt = d.H / 256;
    hipLaunchKernelGGL((grouped_gemm_kernel<false>), dim3(mtiles * nt), dim3(kGemmThreads), 0, st,
                       L, w.act, w.tiles, w.tile_count, w.token_map, w.row_weight, d.A, nt, w.act,
                       w.contrib, call.cap);
  }
  rc = launch_check("grouped down GEMM");
  if (rc != AIMA_OK) return rc;
  if ((rc = record(call.ev[3], st)) != AIMA_OK) return rc;
  if (call.routed_f32) {
    hipLaunchKernelGGL(combine_routed_f32_kernel, dim3((unsigned)d.T), dim3(256), 0, st,
                       w.contrib, w.inverse_map, d.k, (int64_t)d.H, static_cast<float*>(out));
  } else if (d.H == 2048 && d.k <= 8) {
    hipLaunchKernelGGL(combine2048_kernel, dim3((unsigned)d.T), dim3(256), 0, st, w.contrib,
                       w.inverse_map, d.k, d.A, x, L.shared_gate_vec, sigma_in, residual,
                       static_cast<uint16_t*>(out), next);
  } else {
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)d.T), dim3(256), 0, st, w.contrib,
                       w.inverse_map, d.k, d.A, x, L.shared_gate_vec, sigma_in, residual,
                       (int64_t)d.H, static_cast<uint16_t*>(out), next);
  }
  rc = launch_check("grouped combine");
  if (rc != AIMA_OK) return rc;
  return record(call.ev[4], st);
}

// The grouped GEMM addresses its A rows with 32-bit byte offsets.
static bool prefill_offsets_fit(const aima_moe_layer* L, int64_t tokens, int k) {
  const int64_t limit = (int64_t)1 << 30;  // f16 elements (2^31 bytes)
  return tokens * (k + 1) * L->inter < limit && tokens * L->hidden < limit;
}

// need_shared: the call runs the shared expert (every mode but the routed-only
// RunLayer output, which needs no shared tensors).
int check_layer_prefill(const aima_moe_layer* L, int k, bool need_norm, bool need_shared = true) {
  AIMA_REQUIRE(L != nullptr, "moe prefill: null layer");
  AIMA_REQUIRE(L->gate_up.qweight && L->gate_up.scale && L->gate_up.zp && L->down.qweight &&
                   L->down.scale && L->down.zp,
               "moe prefill: null routed tensor pointer");
  AIMA_REQUIRE(!need_shared || (L->shared_gate_up.qweight && L->shared_gate_up.scale &&
                                L->shared_gate_up.zp && L->shared_down.qweight &&
                                L->shared_down.scale && L->shared_down.zp && L->shared_gate_vec),
               "moe prefill: null shared tensor pointer");
  AIMA_REQUIRE(split_tensors_ok(*L),
               "moe prefill: a split up tensor needs qweight, scale and zp (qweight 16-byte aligned)");
  AIMA_REQUIRE(!need_norm || L->norm_weight, "moe prefill: null norm weight");
  AIMA_REQUIRE(L->experts > 0 && L->experts <= kMaxExperts, "moe prefill: experts must be in [1, 1024]");
  AIMA_REQUIRE(k > 0 && k <= 16 && k <= L->experts, "moe prefill: k must be in [1, min(16, experts)]");
  if (L->group != 128) return fail(AIMA_E_UNSUPPORTED, "moe prefill: group must be 128");
  if (need_shared && L->shared_inter != L->inter) {
    return fail(AIMA_E_UNSUPPORTED, "moe prefill: shared_inter must equal inter");
  }
  if (L->hidden % 256 != 0 || L->inter % 128 != 0 || L->hidden <= 0 || L->inter <= 0) {
    return fail(AIMA_E_UNSUPPORTED, "moe prefill: hidden % 256 and inter % 128 must be 0");
  }
  AIMA_REQUIRE(aligned(L->gate_up.qweight, 16) && aligned(L->down.qweight, 16) &&
                   (!need_shared || (aligned(L->shared_gate_up.qweight, 16) &&
                                     aligned(L->shared_down.qweight, 16) &&
                                     aligned(L->shared_gate_vec, 16))),
               "moe prefill: qweight pointers and the shared gate vector must be 16-byte aligned");
  // the stack's fused combine reads the next layer's norm weights as 16-byte vectors
  AIMA_REQUIRE(!need_norm || aligned(L->norm_weight, 16),
               "moe prefill: norm_weight must be 16-byte aligned");
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
  AIMA_REQUIRE(aligned(x, 16) && aligned(out, 16) && (!residual || aligned(residual, 16)),
               "moe_grouped_prefill: x, residual and out must be 16-byte aligned");
  const PrefillDims d = prefill_dims(layer, tokens, k);
  PrefillWs w{};
  const size_t need = prefill_ws_layout(d, WsMode::kLayer, workspace, &w);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "moe_grouped_prefill: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_grouped_prefill: workspace must be 256-byte aligned");
  return prefill_layer(*layer, x, residual, ids, weights, out, d, w, (hipStream_t)stream);
}

extern "C" int aima_moe_grouped_prefill_ex(const aima_moe_layer* layer, const void* x,
                                           const uint16_t* residual, int64_t tokens,
                                           const int32_t* topk, const float* weights, int32_t k,
                                           void* out, const aima_prefill_options* options,
                                           void* workspace, size_t workspace_bytes,
                                           void* stream) {
  aima_prefill_options opt{};
  if (options) opt = *options;
  AIMA_REQUIRE(opt.output_mode == AIMA_PREFILL_FULL_F16 || opt.output_mode == AIMA_PREFILL_ROUTED_F32,
               "moe_grouped_prefill_ex: unknown output mode");
  AIMA_REQUIRE(opt.input_f32 == 0 || opt.input_f32 == 1, "moe_grouped_prefill_ex: input_f32 must be 0 or 1");
  const bool routed = opt.output_mode == AIMA_PREFILL_ROUTED_F32;
  int rc = check_layer_prefill(layer, k, false, !routed);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(x && topk && weights && out, "moe_grouped_prefill_ex: null pointer");
  AIMA_REQUIRE(!routed || !residual,
               "moe_grouped_prefill_ex: the routed-only output takes no residual");
  AIMA_REQUIRE(tokens > 0 && tokens <= (1 << 24), "moe_grouped_prefill_ex: tokens must be in [1, 2^24]");
  // RunLayer requires topk_stride >= 8 * sizeof(int32) for its top-8
  // (grouped_s8_u4_prefill_runtime.cpp:1044-1045); here >= k * 4
  const int64_t stride_bytes = opt.topk_stride ? opt.topk_stride : (int64_t)k * 4;
  AIMA_REQUIRE(stride_bytes >= (int64_t)k * 4 && stride_bytes % 4 == 0 &&
                   stride_bytes / 4 <= (1 << 20),
               "moe_grouped_prefill_ex: topk_stride must be a multiple of 4, >= 4 * k and <= 4 MiB");
  AIMA_REQUIRE(aligned(topk, 4), "moe_grouped_prefill_ex: topk must be 4-byte aligned");
  AIMA_REQUIRE(prefill_offsets_fit(layer, tokens, k),
               "moe_grouped_prefill_ex: tokens * (k + 1) * inter and tokens * hidden must stay "
               "below 2^30 (split the batch)");
  AIMA_REQUIRE(aligned(x, 16) && aligned(out, 16) && (!residual || aligned(residual, 16)),
               "moe_grouped_prefill_ex: x, residual and out must be 16-byte aligned");
  const PrefillDims d = prefill_dims(layer, tokens, k);
  PrefillWs w{};
  const size_t need = prefill_ws_layout(d, WsMode::kLayer, workspace, &w);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "moe_grouped_prefill_ex: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_grouped_prefill_ex: workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  LayerCall call;
  call.stride = (int)(stride_bytes / 4);
  call.routed_f32 = routed;
  for (int i = 0; i < 5; ++i) call.ev[i] = static_cast<hipEvent_t>(opt.stage_events[i]);
  AIMA_REQUIRE(aligned(opt.swiglu_f32, 16) && aligned(opt.contributions_f32, 16),
               "moe_grouped_prefill_ex: the f32 capture buffers must be 16-byte aligned");
  call.cap = GemmCapture{opt.swiglu_f32, opt.contributions_f32};
  const uint16_t* x16 = static_cast<const uint16_t*>(x);
  if (opt.input_f32) {
    const int64_t n8 = tokens * layer->hidden / 8;
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st,
                       static_cast<const float4*>(x), n8, reinterpret_cast<u32x4*>(w.x16));
    rc = launch_check("moe_grouped_prefill_ex input conversion");
    if (rc != AIMA_OK) return rc;
    x16 = w.x16;
  }
  return prefill_layer(*layer, x16, residual, topk, weights, out, d, w, st, nullptr,
                       CombineNext{}, call);
}

// MOE3GemmFusedCompressed's operation: router logits in, the selection of
// select_router_topk per token (the router top-k kernel, ids and weights into
// the caller's buffers), then the grouped layer of aima_moe_grouped_prefill_ex
// on those dense routes.
extern "C" int aima_moe_grouped_prefill_logits(const aima_moe_layer* layer, const void* x,
                                               const uint16_t* residual, int64_t tokens,
                                               const float* routing_logits, int32_t k,
                                               float min_weight_sum, int32_t* ids_out,
                                               float* weights_out, void* out,
                                               const aima_prefill_options* options,
                                               void* workspace, size_t workspace_bytes,
                                               void* stream) {
  AIMA_REQUIRE(layer && x && routing_logits && ids_out && weights_out && out,
               "moe_grouped_prefill_logits: null pointer");
  aima_prefill_options opt{};
  if (options) opt = *options;
  AIMA_REQUIRE(opt.topk_stride == 0 || opt.topk_stride == (int64_t)k * 4,
               "moe_grouped_prefill_logits: the routes are dense (topk_stride 0)");
  AIMA_REQUIRE(tokens > 0 && tokens <= (1 << 24),
               "moe_grouped_prefill_logits: tokens must be in [1, 2^24]");
  // everything the layer call checks, before the selection is launched
  int rc = check_layer_prefill(layer, k, false, opt.output_mode != AIMA_PREFILL_ROUTED_F32);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(min_weight_sum > 0.f,
               "moe_grouped_prefill_logits: minimum weight sum must be positive");
  const PrefillDims d = prefill_dims(layer, tokens, k);
  if (!workspace || workspace_bytes < prefill_ws_layout(d, WsMode::kLayer, nullptr, nullptr)) {
    return fail(AIMA_E_WORKSPACE, "moe_grouped_prefill_logits: workspace missing or too small");
  }
  const hipStream_t st = (hipStream_t)stream;
  hipEvent_t first = static_cast<hipEvent_t>(opt.stage_events[0]);
  if ((rc = record(first, st)) != AIMA_OK) return rc;
  opt.stage_events[0] = nullptr;  // event 0 marks the start of the selection
  rc = aima_router_topk(routing_logits, tokens, layer->experts, k, min_weight_sum, ids_out,
                        weights_out, stream);
  if (rc != AIMA_OK) return rc;
  opt.topk_stride = 0;
  return aima_moe_grouped_prefill_ex(layer, x, residual, tokens, ids_out, weights_out, k, out,
                                     &opt, workspace, workspace_bytes, stream);
}

extern "C" int aima_moe_prefill_workspace_views(const aima_moe_layer* layer, int64_t tokens,
                                                int32_t k, void* workspace,
                                                aima_prefill_views* views) {
  AIMA_REQUIRE(layer && workspace && views, "moe_prefill_workspace_views: null pointer");
  AIMA_REQUIRE(tokens > 0 && k > 0, "moe_prefill_workspace_views: tokens and k must be positive");
  PrefillWs w{};
  prefill_ws_layout(prefill_dims(layer, tokens, k), WsMode::kLayer, workspace, &w);
  views->offsets = w.offsets;
  views->token_map = w.token_map;
  views->inverse_map = w.inverse_map;
  views->compact_weights = w.row_weight;
  views->swiglu = w.act;
  views->contributions = w.contrib;
  views->tiles = w.tiles;
  views->tile_count = w.tile_count;
  return AIMA_OK;
}

extern "C" int aima_moe_stack_prefill(const aima_moe_layer* layers, int32_t n_layers, float eps,
                                      const uint16_t* x_in, int64_t tokens, const int32_t* ids,
                                      const float* weights, int32_t k, uint16_t* out,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  AIMA_REQUIRE(layers && n_layers > 0, "moe_stack_prefill: need at least one layer");
  AIMA_REQUIRE(x_in && ids && weights && out, "moe_stack_prefill: null pointer");
  AIMA_REQUIRE(aligned(x_in, 16) && aligned(out, 16),
               "moe_stack_prefill: x and out must be 16-byte aligned");
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
  // layer 0's normalized input comes from the rmsnorm kernel; every later
  // one (and its shared-expert gate) from the previous layer's combine
  int rc = rmsnorm_launch(r, layers[0].norm_weight, tokens, layers[0].hidden, eps, w.h, st);
  if (rc != AIMA_OK) return rc;
  for (int32_t l = 0; l < n_layers; ++l) {
    const aima_moe_layer& L = layers[l];
    uint16_t* dst = (l == n_layers - 1) ? out : w.r[l & 1];
    CombineNext next{};
    if (l + 1 < n_layers) {
      next.norm = layers[l + 1].norm_weight;
      next.gate_vec = layers[l + 1].shared_gate_vec;
      next.eps = eps;
      next.h = w.h;  // each block rewrites only its own row, after reading it
      next.sigma = w.sigma[(l + 1) & 1];
    }
    rc = prefill_layer(L, w.h, r, ids + (int64_t)l * d.A, weights + (int64_t)l * d.A, dst, d, w,
                       st, l > 0 ? w.sigma[l & 1] : nullptr, next);
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
  int rc = launch_schedule(ids, k, weights, d, w, true, st);
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
