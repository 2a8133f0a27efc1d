// Device top-k over f32 values and the U4 LM head with top-k, for gfx950.
//
// Order: value descending, the lower index first among equal values -- the
// order of the reference's LM-head partial top-8 (q4x8_matvec.cl:973-1021:
// an insertion that keeps an earlier index ahead of an equal later value).
// NaN values are never chosen; with fewer than k numbers the remaining
// ranks hold the empty pair (-inf, 0x7fffffff).
//
// One launch.  P <= 256 blocks of 1024 threads; block b owns a contiguous
// chunk of at most 4096 values (4 per thread) and selects its k best
// (block_select) into its partial slots.  The block that arrives last at a
// device-scope counter in the workspace header selects the final k from
// the P * k partials (see topk_kernel for how it knows they are all
// written) and clears the counter.  P = 1 writes the result directly.
// n <= 1,048,576.
//
// The LM head (aima_u4_lm_head_topk) is the U4 matvec into the caller's
// logits followed by this selection.  A variant with the reference's shape
// -- every matvec block writing its own partial top-k, the selection then
// running over those candidates -- measured slower: the block barrier and
// ranking in each of the 7,760 matvec blocks cost 5.6 us at N = 248,320,
// while the selection is bound by latency, not by the 1 MB of logits it
// reads.
#include "common.h"

#include <math.h>

namespace aima {

int u4_matvec_dispatch(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                       const uint8_t* zp, int64_t n, int64_t k, int glog2, void* y,
                       int out_f32, hipStream_t st);
int group_log2_of(int group);

namespace {

constexpr int kTopkMax = 16;
constexpr int kNoIndex = 0x7fffffff;
constexpr int kPassThreads = 1024;
constexpr int kPerThread = 4;
constexpr int kMaxPartials = 256;
constexpr int64_t kChunkMax = (int64_t)kPassThreads * kPerThread;
constexpr int64_t kTopkMaxN = kChunkMax * kMaxPartials;
constexpr int kWaves = kPassThreads / 64;
constexpr int kMaxCand = 256;  // candidates one wave selects from (4 per lane)

// The selection's block counter and epoch, kept in the workspace header at
// byte 128 (the error word is at 0): the counter is zero in a fresh
// (zero-filled) workspace and the last block of every launch leaves it zero
// again; the epoch (any start value) advances by one per launch.
constexpr size_t kTopkCounterOffset = 128;

__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  return av > bv || (av == bv && ai < bi);
}

// k rounds of a wave-wide maximum over PER candidates per lane; lane r ends
// holding the rank-r pick (r < k).  Once the real candidates run out the
// picks are the empty pair.
template <int PER>
__device__ __forceinline__ void wave_topk(float (&v)[PER], int (&ix)[PER], int k, float& out_v,
                                          int& out_i) {
  const int lane = threadIdx.x & 63;
  out_v = -INFINITY;
  out_i = kNoIndex;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = kNoIndex;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (better(v[j], ix[j], bv, bi)) {
        bv = v[j];
        bi = ix[j];
      }
    }
    wave_best_pair(bv, bi);
    if (lane == r) {
      out_v = bv;
      out_i = bi;
    }
    // the pick leaves the candidate set (indices are unique)
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (ix[j] == bi) {
        v[j] = -INFINITY;
        ix[j] = kNoIndex;
      }
    }
  }
}

struct SelectLds {
  float v[kWaves * kTopkMax];
  int i[kWaves * kTopkMax];
  float wv[kWaves];
  int wi[kWaves];
  int cnt[kWaves];
  float cv[kMaxCand];
  int ci[kMaxCand];
  int is_last;
};

// The block's top-k of PER (value, index) pairs per thread; wave 0 lanes
// r < k write rank r to out_v / out_i.  Every thread of the block calls it.
//
// Threshold filter first: each wave finds its best pair; the k-th best of
// the 16 wave bests, T, bounds the block's top-k from below (the k wave
// bests at or above T are k pairs at least as good), so only pairs at or
// above T can be picked.  They are compacted into LDS (ballots give each its
// slot).  Up to 64 of them (the usual case: the 16 wave bests and a few
// more): lane l ranks survivor l against all of them and the survivor of
// rank r < k is pick r.  Up to 256: wave 0 selects by k rounds of a
// wave-wide maximum.  When ties leave more than 256, every wave selects its
// own k and wave 0 merges the 16 lists.
template <int PER>
__device__ void block_select(float (&v)[PER], int (&ix)[PER], int k, SelectLds& S, float* out_v,
                             int32_t* out_i) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // wave bests
  float bv = -INFINITY;
  int bi = kNoIndex;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (better(v[j], ix[j], bv, bi)) {
      bv = v[j];
      bi = ix[j];
    }
  }
  wave_best_pair(bv, bi);
  if (lane == 0) {
    S.wv[wave] = bv;
    S.wi[wave] = bi;
  }
  __syncthreads();
  // T = the k-th best wave best: lane w < 16 ranks wave best w against all 16
  float tv = -INFINITY;
  int ti = kNoIndex;
  {
    int rank = kWaves;
    float mv = -INFINITY;
    int mi = kNoIndex;
    if (lane < kWaves) {
      mv = S.wv[lane];
      mi = S.wi[lane];
      rank = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) rank += better(S.wv[w], S.wi[w], mv, mi) ? 1 : 0;
    }
    // no rank k-1 (fewer than k waves hold values, their empty bests tie):
    // no filter, every valid pair qualifies
    const uint64_t hit = __ballot(rank == k - 1);
    if (hit) {
      const int src = (int)__builtin_ctzll(hit);
      tv = lane_read(mv, src);
      ti = __builtin_amdgcn_readlane(mi, src);
    }
  }
  // compact the pairs at or above T
  int cnt = 0;
  bool q[PER];
  uint64_t mask[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    q[j] = ix[j] != kNoIndex && (better(v[j], ix[j], tv, ti) || (v[j] == tv && ix[j] == ti));
    mask[j] = __ballot(q[j]);
    cnt += __builtin_popcountll(mask[j]);
  }
  if (lane == 0) S.cnt[wave] = cnt;
  __syncthreads();
  int wbase = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = S.cnt[w];
    wbase += w < wave ? c : 0;
    total += c;
  }
  if (total <= kMaxCand) {
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int off = wbase;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (q[j]) {
        const int slot = off + __builtin_popcountll(mask[j] & below);
        S.cv[slot] = v[j];
        S.ci[slot] = ix[j];
      }
      off += __builtin_popcountll(mask[j]);
    }
    __syncthreads();
    if (wave != 0) return;
    if (total <= 64) {
      const bool mine = lane < total;
      const float mv = mine ? S.cv[lane] : -INFINITY;
      const int mi = mine ? S.ci[lane] : kNoIndex;
      int rank = 0;
      for (int j = 0; j < total; ++j) rank += better(S.cv[j], S.ci[j], mv, mi) ? 1 : 0;
      if (mine && rank < k) {
        out_v[rank] = mv;
        out_i[rank] = mi;
      }
      if (lane >= total && lane < k) {  // fewer than k numbers in the block
        out_v[lane] = -INFINITY;
        out_i[lane] = kNoIndex;
      }
      return;
    }
    float c[kMaxCand / 64];
    int ci[kMaxCand / 64];
#pragma unroll
    for (int j = 0; j < kMaxCand / 64; ++j) {
      const int slot = lane + 64 * j;
      c[j] = slot < total ? S.cv[slot] : -INFINITY;
      ci[j] = slot < total ? S.ci[slot] : kNoIndex;
    }
    float wv;
    int wi;
    wave_topk<kMaxCand / 64>(c, ci, k, wv, wi);
    if (lane < k) {
      out_v[lane] = wv;
      out_i[lane] = wi;
    }
    return;
  }
  // many ties at the threshold: per-wave selection, then a merge
  float wv;
  int wi;
  wave_topk<PER>(v, ix, k, wv, wi);
  if (lane < k) {
    S.v[wave * k + lane] = wv;
    S.i[wave * k + lane] = wi;
  }
  __syncthreads();
  if (wave == 0) {
    constexpr int kCandPer = kWaves * kTopkMax / 64;
    float c[kCandPer];
    int ci[kCandPer];
#pragma unroll
    for (int j = 0; j < kCandPer; ++j) {
      const int qi = lane + 64 * j;
      c[j] = qi < kWaves * k ? S.v[qi] : -INFINITY;
      ci[j] = qi < kWaves * k ? S.i[qi] : kNoIndex;
    }
    wave_topk<kCandPer>(c, ci, k, wv, wi);
    if (lane < k) {
      out_v[lane] = wv;
      out_i[lane] = wi;
    }
  }
}

// A partial pick as one 64-bit word: the value's bits, then 21 bits of
// index (0x1fffff = none) and 11 bits of the launch's epoch, so a reader
// can tell a slot written by this launch from a stale one.
constexpr uint32_t kNoIndex21 = 0x1fffffu;
__device__ __forceinline__ uint64_t pack_pick(float v, int ix, uint32_t epoch) {
  const uint32_t i21 = ix == kNoIndex ? kNoIndex21 : (uint32_t)ix;
  return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)(i21 | (epoch << 21)) << 32);
}
constexpr uint32_t kSpinLimit = 1u << 22;

// The selection (see the file comment).  state: the workspace header's
// counter and epoch words; partial: P * k packed picks (both unused when
// P = 1).  Every block reads the epoch the previous launch left, stores its
// partial picks tagged with it (device scope), waits for those stores and
// then takes a ticket from the counter.  The block with the last ticket
// also checks that every partial slot carries the epoch (device-scope
// loads, repeated until they do; a spin limit sets AIMA_DEVERR_TIMEOUT in
// the error word), selects, and leaves counter 0 and the next epoch.  No
// device-wide cache write-back or invalidate is involved (a __threadfence
// per block made the selection take 70 us instead of a few).
__global__ __launch_bounds__(kPassThreads) void topk_kernel(
    const float* __restrict__ vals, int64_t n, int64_t chunk, int k, uint64_t* __restrict__ partial,
    uint32_t* __restrict__ state, float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  __shared__ SelectLds S;
  __shared__ float pick_v[kTopkMax];
  __shared__ int32_t pick_i[kTopkMax];
  const int64_t base = (int64_t)blockIdx.x * chunk;
  const int64_t end = base + chunk < n ? base + chunk : n;
  uint32_t* const err = state;  // the workspace error word (byte 0)
  uint32_t* const counter = state + kTopkCounterOffset / 4;
  uint32_t* const epoch_word = counter + 1;
  uint32_t epoch = 0;
  if (gridDim.x > 1) {
    epoch = __hip_atomic_load(epoch_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 0x7ffu;
  }
  float v[kPerThread];
  int ix[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    // positions past the chunk read its last element (straight-line loads,
    // all in flight at once) and are then emptied
    const int64_t p = base + threadIdx.x + (int64_t)kPassThreads * j;
    const int64_t pc = p < end ? p : end - 1;
    const float val = vals[pc];
    v[j] = p < end ? val : -INFINITY;
    ix[j] = p < end ? (int)p : kNoIndex;
  }
  if (gridDim.x == 1) {
    block_select<kPerThread>(v, ix, k, S, out_v, out_i);
    return;
  }
  block_select<kPerThread>(v, ix, k, S, pick_v, pick_i);
  __syncthreads();
  if ((int)threadIdx.x < k) {
    __hip_atomic_store(&partial[(int64_t)blockIdx.x * k + threadIdx.x],
                       pack_pick(pick_v[threadIdx.x], pick_i[threadIdx.x], epoch),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (threadIdx.x == 0) {
    // the picks are stored by lanes of this wave: let them complete first
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    S.is_last = atomicAdd(counter, 1u) == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (!S.is_last) return;
  const int np = (int)gridDim.x * k;  // <= 256 * 16 = 4096
  uint64_t w[kPerThread];
  for (uint32_t spins = 0;; ++spins) {
    bool fresh = true;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int q = (int)threadIdx.x + kPassThreads * j;
      const int qc = q < np ? q : np - 1;
      w[j] = __hip_atomic_load(&partial[qc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      fresh = fresh && (uint32_t)(w[j] >> 53) == epoch;
    }
    if (__syncthreads_and(fresh)) break;
    if (spins > kSpinLimit) {
      if (threadIdx.x == 0) atomicOr(err, AIMA_DEVERR_TIMEOUT);
      break;
    }
  }
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int q = (int)threadIdx.x + kPassThreads * j;
    const uint32_t i21 = (uint32_t)(w[j] >> 32) & kNoIndex21;
    v[j] = q < np ? __builtin_bit_cast(float, (uint32_t)w[j]) : -INFINITY;
    ix[j] = q < np && i21 != kNoIndex21 ? (int)i21 : kNoIndex;
  }
  block_select<kPerThread>(v, ix, k, S, out_v, out_i);
  if (threadIdx.x == 0) {
    *counter = 0u;
    *epoch_word = (epoch + 1u) & 0x7ffu;
  }
}

int partial_blocks(int64_t n) {
  const int64_t p = (n + kPassThreads - 1) / kPassThreads;
  return (int)(p < kMaxPartials ? p : kMaxPartials);
}

// Workspace: the header (error word at 0, counter and epoch at
// kTopkCounterOffset), then the P * k packed partial picks.
size_t topk_ws_bytes(int64_t n, int k) {
  return kWsHeader + round_up((size_t)partial_blocks(n) * k * 8, 256);
}

int topk_launch(const float* values, int64_t n, int k, int32_t* ids, float* out_values, void* ws,
                size_t ws_bytes, hipStream_t st) {
  const int P = partial_blocks(n);
  const int64_t chunk = (n + P - 1) / P;
  uint64_t* partial = nullptr;
  uint32_t* state = nullptr;
  if (P > 1) {
    AIMA_REQUIRE(ws && aligned(ws, 256) && ws_bytes >= topk_ws_bytes(n, k),
                 "topk: workspace missing, unaligned or too small");
    state = static_cast<uint32_t*>(ws);
    partial = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsHeader);
  }
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)P), dim3(kPassThreads), 0, st, values, n, chunk,
                     k, partial, state, out_values, ids);
  return launch_check("topk");
}

int check_topk_args(int64_t n, int32_t k) {
  AIMA_REQUIRE(n > 0 && n <= kTopkMaxN, "topk: n must be in [1, 1048576]");
  AIMA_REQUIRE(k > 0 && k <= kTopkMax && k <= n, "topk: k must be in [1, min(16, n)]");
  return AIMA_OK;
}

}  // namespace
}  // namespace aima

using namespace aima;

extern "C" int aima_topk_workspace_size(int64_t n, int32_t k, size_t* bytes) {
  AIMA_REQUIRE(bytes, "topk_workspace_size: null pointer");
  const int rc = check_topk_args(n, k);
  if (rc != AIMA_OK) return rc;
  *bytes = topk_ws_bytes(n, k);
  return AIMA_OK;
}

extern "C" int aima_topk_f32(const float* values, int64_t n, int32_t k, int32_t* ids,
                             float* out_values, void* workspace, size_t workspace_bytes,
                             void* stream) {
  AIMA_REQUIRE(values && ids && out_values, "topk: null pointer");
  const int rc = check_topk_args(n, k);
  if (rc != AIMA_OK) return rc;
  return topk_launch(values, n, k, ids, out_values, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int aima_u4_lm_head_topk(const uint16_t* x, const uint8_t* qweight,
                                    const uint16_t* scale, const uint8_t* zp, int64_t n,
                                    int64_t k, int32_t group, int32_t topk, float* logits,
                                    int32_t* ids, float* values, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  AIMA_REQUIRE(x && qweight && scale && zp && logits && ids && values,
               "lm_head_topk: null pointer");
  int rc = check_topk_args(n, topk);
  if (rc != AIMA_OK) return rc;
  const int glog2 = group_log2_of(group);
  AIMA_REQUIRE(glog2 > 0, "lm_head_topk: group must be 32, 64, 128 or 256");
  AIMA_REQUIRE(k % group == 0, "lm_head_topk: k must be a multiple of group");
  AIMA_REQUIRE(aligned(qweight, 16) && aligned(x, 16),
               "lm_head_topk: qweight and x must be 16-byte aligned");
  AIMA_REQUIRE(partial_blocks(n) == 1 ||
                   (workspace && aligned(workspace, 256) &&
                    workspace_bytes >= topk_ws_bytes(n, topk)),
               "lm_head_topk: workspace missing, unaligned or too small");
  const hipStream_t st = (hipStream_t)stream;
  rc = u4_matvec_dispatch(x, qweight, scale, zp, n, k, glog2, logits, 1, st);
  if (rc != AIMA_OK) return rc;
  return topk_launch(logits, n, topk, ids, values, workspace, workspace_bytes, st);
}
