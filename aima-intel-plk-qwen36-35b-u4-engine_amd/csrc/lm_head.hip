// Device top-k over f32 values and the U4 LM head with top-k, for gfx950.
//
// Order: value descending, the lower index first among equal values -- the
// order of the reference's LM-head partial top-8 (q4x8_matvec.cl:973-1021:
// an insertion that keeps an earlier index ahead of an equal later value).
// NaN values are never chosen; with fewer than k numbers the remaining
// ranks hold the empty pair (-inf, 0x7fffffff).
//
// One launch.  P <= 256 blocks of 256 threads (one wave per SIMD); block b
// owns a contiguous chunk of at most 4096 values (16 per thread) and selects
// its k best (block_select) into its partial slots.  Block 0 then selects
// the final k from the P * k partials once every slot carries the launch's
// tags (see topk_kernel).  P = 1 writes the result directly.
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
constexpr int kPassThreads = 256;
constexpr int kPerThread = 16;  // the final selection: P * k <= 256 * 16 picks
constexpr int kMaxPartials = 256;
constexpr int64_t kChunkMax = (int64_t)kPassThreads * kPerThread;
constexpr int64_t kTopkMaxN = kChunkMax * kMaxPartials;

constexpr int kWaves = kPassThreads / 64;
constexpr int kRowBests = kWaves * 4;  // one best per 16-lane row
static_assert(kRowBests >= kTopkMax, "the threshold needs k row bests");
constexpr int kMaxCand = 256;  // candidates one wave selects from (4 per lane)

// The selection's launch counter, kept in the workspace header at byte 132
// (the error word is at 0; bytes 128..131 stay zero): any start value, and
// it advances by one per launch.  A launch tags both words of each of its
// picks with the full 32-bit counter value (see pick_value_word), so a slot
// is taken only when it was written by this launch: a zero-filled slot, a
// slot of an earlier launch and data other entry points left in the same
// memory all fail the check (short of matching two 32-bit tags at once).
constexpr size_t kTopkLaunchOffset = 132;

// (bitwise on the comparisons: no short-circuit branches)
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  return (av > bv) | ((av == bv) & (ai < bi));
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
  alignas(16) float rv[kRowBests];
  alignas(16) int ri[kRowBests];
  int count;
  alignas(16) float cv[kMaxCand];
  alignas(16) int ci[kMaxCand];
};

// The block's top-k of PER (value, index) pairs per thread; wave 0 lanes
// r < k write rank r to out_v / out_i.  Every thread of the block calls it.
//
// Threshold filter first: every 16-lane row finds its best pair (DPP inside
// the row); the k-th best of the 16 row bests, T, bounds the block's top-k
// from below (the k row bests at or above T are k pairs at least as good),
// so only pairs at or above T can be picked.  Those few are appended to LDS
// through an LDS counter (their order does not matter: they are ranked by
// (value, index) next).  Up to 64 of them (the usual case: about the 16 row
// bests): lane l ranks survivor l against all of them and the survivor of
// rank r < k is pick r.  Up to 256: wave 0 selects by k rounds of a
// wave-wide maximum.  When ties leave more than 256, every wave selects its
// own k and wave 0 merges the lists.
template <int PER>
__device__ void block_select(float (&v)[PER], int (&ix)[PER], int k, SelectLds& S, float* out_v,
                             int32_t* out_i) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // row bests: the lane's best by a pairwise tree (independent compares at
  // each level, not one chain of PER), then DPP inside the row
  static_assert((PER & (PER - 1)) == 0, "PER is a power of two");
  float tv_[PER];
  int ti_[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    // NaN is never chosen: it becomes the empty pair (a NaN kept in the
    // tree would beat nothing and hide the lane's real values); selects,
    // not a branch, so the arrays stay in place
    const bool nan = v[j] != v[j];
    ix[j] = nan ? kNoIndex : ix[j];
    v[j] = nan ? -INFINITY : v[j];
    tv_[j] = v[j];
    ti_[j] = ix[j];
  }
#pragma unroll
  for (int w = PER / 2; w > 0; w /= 2) {
#pragma unroll
    for (int j = 0; j < w; ++j) {
      const bool b = better(tv_[j + w], ti_[j + w], tv_[j], ti_[j]);
      tv_[j] = b ? tv_[j + w] : tv_[j];
      ti_[j] = b ? ti_[j + w] : ti_[j];
    }
  }
  const float lane_v = tv_[0];
  const int lane_i = ti_[0];
  float bv = lane_v;
  int bi = lane_i;
  pair_step<0xB1>(bv, bi);   // quad_perm [1,0,3,2]
  pair_step<0x4E>(bv, bi);   // quad_perm [2,3,0,1]
  pair_step<0x141>(bv, bi);  // row_half_mirror
  pair_step<0x140>(bv, bi);  // row_mirror
  if ((lane & 15) == 0) {
    S.rv[wave * 4 + (lane >> 4)] = bv;
    S.ri[wave * 4 + (lane >> 4)] = bi;
  }
  if (threadIdx.x == 0) S.count = 0;
  __syncthreads();
  // T = the k-th best row best: lane r < 16 ranks row best r against all 16
  float tv = -INFINITY;
  int ti = kNoIndex;
  {
    int rank = kRowBests;
    float mv = -INFINITY;
    int mi = kNoIndex;
    if (lane < kRowBests) {
      mv = S.rv[lane];
      mi = S.ri[lane];
      rank = 0;
#pragma unroll
      for (int w = 0; w < kRowBests; w += 4) {
        const float4 a = *reinterpret_cast<const float4*>(&S.rv[w]);
        const int4 ia = *reinterpret_cast<const int4*>(&S.ri[w]);
        rank += (better(a.x, ia.x, mv, mi) ? 1 : 0) + (better(a.y, ia.y, mv, mi) ? 1 : 0) +
                (better(a.z, ia.z, mv, mi) ? 1 : 0) + (better(a.w, ia.w, mv, mi) ? 1 : 0);
      }
    }
    // no rank k-1 (fewer than k rows hold values, their empty bests tie):
    // no filter, every valid pair qualifies
    const uint64_t hit = __ballot(rank == k - 1);
    if (hit) {
      const int src = (int)__builtin_ctzll(hit);
      tv = lane_read(mv, src);
      ti = __builtin_amdgcn_readlane(mi, src);
    }
  }
  // append the pairs at or above T (few: a lane whose own best is below T
  // holds none, so only the lanes that do scan their values)
  auto at_or_above = [&](float pv, int pi) {
    return (pi != kNoIndex) & ((pv > tv) | ((pv == tv) & (pi <= ti)));
  };
  if (at_or_above(lane_v, lane_i)) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (at_or_above(v[j], ix[j])) {
        const int slot = atomicAdd(&S.count, 1);
        if (slot < kMaxCand) {
          S.cv[slot] = v[j];
          S.ci[slot] = ix[j];
        }
      }
    }
  }
  __syncthreads();
  const int total = S.count;
  if (total <= kMaxCand) {
    if (wave != 0) return;
    if (total <= 64) {
      const bool mine = lane < total;
      const float mv = mine ? S.cv[lane] : -INFINITY;
      const int mi = mine ? S.ci[lane] : kNoIndex;
      // survivors padded with empty pairs to a multiple of 8, then compared
      // eight at a time from 16-byte LDS reads (every lane reads the same
      // words), so the reads are in flight together
      const int tot8 = (total + 7) & ~7;
      if (lane >= total && lane < tot8) {
        S.cv[lane] = -INFINITY;
        S.ci[lane] = kNoIndex;
      }
      wave_lds_sync();
      int rank = 0;
      for (int j = 0; j < tot8; j += 8) {
        const float4 a = *reinterpret_cast<const float4*>(&S.cv[j]);
        const float4 b = *reinterpret_cast<const float4*>(&S.cv[j + 4]);
        const int4 ia = *reinterpret_cast<const int4*>(&S.ci[j]);
        const int4 ib = *reinterpret_cast<const int4*>(&S.ci[j + 4]);
        rank += (better(a.x, ia.x, mv, mi) ? 1 : 0) + (better(a.y, ia.y, mv, mi) ? 1 : 0) +
                (better(a.z, ia.z, mv, mi) ? 1 : 0) + (better(a.w, ia.w, mv, mi) ? 1 : 0) +
                (better(b.x, ib.x, mv, mi) ? 1 : 0) + (better(b.y, ib.y, mv, mi) ? 1 : 0) +
                (better(b.z, ib.z, mv, mi) ? 1 : 0) + (better(b.w, ib.w, mv, mi) ? 1 : 0);
      }
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
    constexpr int kCandPer = (kWaves * kTopkMax + 63) / 64;
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

// A partial pick as two 64-bit words, each stored and loaded whole: the
// value's bits with the launch number, and the index with the launch number
// xor kTagMix.  Each word validates itself; a slot is fresh when both carry
// this launch's tags.  (kTagMix is non-zero, so an all-zero slot never
// passes, whatever the counter.)
constexpr uint32_t kTagMix = 0x5bd1e995u;
__device__ __forceinline__ uint64_t pick_value_word(float v, uint32_t launch) {
  return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)launch << 32);
}
__device__ __forceinline__ uint64_t pick_index_word(int ix, uint32_t launch) {
  return (uint64_t)(uint32_t)ix | ((uint64_t)(launch ^ kTagMix) << 32);
}
constexpr uint32_t kSpinLimit = 1u << 22;

// The final selection over the P * k packed picks, FPER per thread.
template <int FPER>
__device__ void select_partials(const uint64_t (&wv)[kPerThread],
                                const uint64_t (&wi)[kPerThread], int np, int k, SelectLds& S,
                                float* out_v, int32_t* out_i) {
  float fv[FPER];
  int fix[FPER];
#pragma unroll
  for (int j = 0; j < FPER; ++j) {
    const int q = (int)threadIdx.x + kPassThreads * j;
    fv[j] = q < np ? __builtin_bit_cast(float, (uint32_t)wv[j]) : -INFINITY;
    fix[j] = q < np ? (int)(uint32_t)wi[j] : kNoIndex;
  }
  block_select<FPER>(fv, fix, k, S, out_v, out_i);
}

// The selection (see the file comment).  state: the workspace header (the
// error word, then the launch counter at kTopkLaunchOffset); partial: P * k
// picks of two words each (both unused when P = 1).  Every block reads the
// counter the previous launch left and stores its picks tagged with it
// (device-scope stores); block 0 then reads all P * k slots (device-scope
// loads) until every word carries this launch's tag -- a spin limit sets
// AIMA_DEVERR_TIMEOUT in the error word -- selects the final k and advances
// the counter.  No block
// waits for its own stores, takes a ticket or writes back or invalidates a
// cache (a __threadfence per block made the selection take 70 us instead of
// a few; a ticket counter costs every block a store and an atomic round
// trip).  All P <= 256 blocks are resident together, so block 0's wait ends.
template <int PER>
__global__ __launch_bounds__(kPassThreads) void topk_kernel(
    const float* __restrict__ vals, int64_t n, int64_t chunk, int k, uint64_t* __restrict__ partial,
    uint32_t* __restrict__ state, float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  __shared__ SelectLds S;
  __shared__ float pick_v[kTopkMax];
  __shared__ int32_t pick_i[kTopkMax];
  const int64_t base = (int64_t)blockIdx.x * chunk;
  const int64_t end = base + chunk < n ? base + chunk : n;
  uint32_t* const err = state;  // the workspace error word (byte 0)
  uint32_t* const epoch_word = state + kTopkLaunchOffset / 4;
  uint32_t launch = 0;
  if (gridDim.x > 1) {
    launch = __hip_atomic_load(epoch_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  float v[PER];
  int ix[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    // positions past the chunk read its last element (straight-line loads,
    // all in flight at once) and are then emptied
    const int64_t p = base + threadIdx.x + (int64_t)kPassThreads * j;
    const int64_t pc = p < end ? p : end - 1;
    const float val = vals[pc];
    v[j] = p < end ? val : -INFINITY;
    ix[j] = p < end ? (int)p : kNoIndex;
  }
  if (gridDim.x == 1) {
    block_select<PER>(v, ix, k, S, out_v, out_i);
    return;
  }
  block_select<PER>(v, ix, k, S, pick_v, pick_i);
  __syncthreads();
  if ((int)threadIdx.x < k) {
    uint64_t* slot = partial + 2 * ((int64_t)blockIdx.x * k + threadIdx.x);
    __hip_atomic_store(slot, pick_value_word(pick_v[threadIdx.x], launch), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(slot + 1, pick_index_word(pick_i[threadIdx.x], launch),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (blockIdx.x != 0) return;
  const int np = (int)gridDim.x * k;  // <= 256 * 16 = 4096
  const uint32_t tag_i = launch ^ kTagMix;
  uint64_t wv[kPerThread], wi[kPerThread];
  const int fper = np <= 2 * kPassThreads ? 2 : np <= 4 * kPassThreads ? 4
                   : np <= 8 * kPassThreads ? 8 : 16;
  for (uint32_t spins = 0;; ++spins) {
    bool fresh = true;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int q = (int)threadIdx.x + kPassThreads * j;
      if (j < fper) {
        const int qc = q < np ? q : np - 1;
        wv[j] = __hip_atomic_load(&partial[2 * qc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wi[j] = __hip_atomic_load(&partial[2 * qc + 1], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        fresh = fresh && (uint32_t)(wv[j] >> 32) == launch && (uint32_t)(wi[j] >> 32) == tag_i;
      } else {
        wv[j] = 0;
        wi[j] = 0;
      }
    }
    if (__syncthreads_and(fresh)) break;
    if (spins > kSpinLimit) {
      if (threadIdx.x == 0) atomicOr(err, AIMA_DEVERR_TIMEOUT);
      break;
    }
  }
  if (fper == 2) {
    select_partials<2>(wv, wi, np, k, S, out_v, out_i);
  } else if (fper == 4) {
    select_partials<4>(wv, wi, np, k, S, out_v, out_i);
  } else if (fper == 8) {
    select_partials<8>(wv, wi, np, k, S, out_v, out_i);
  } else {
    select_partials<16>(wv, wi, np, k, S, out_v, out_i);
  }
  // device scope, like the loads that read it: the next launch's blocks
  // (on any XCD) must see the new counter, never this launch's
  if (threadIdx.x == 0) {
    __hip_atomic_store(epoch_word, launch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

int partial_blocks(int64_t n) {
  const int64_t p = (n + kChunkMax - 1) / kChunkMax;
  return (int)(p < kMaxPartials ? p : kMaxPartials);
}

// Workspace: the header (error word at 0, launch counter at
// kTopkLaunchOffset), then the P * k partial picks, 16 bytes each.
size_t topk_ws_bytes(int64_t n, int k) {
  return kWsHeader + round_up((size_t)partial_blocks(n) * k * 16, 256);
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
  hipLaunchKernelGGL(topk_kernel<kPerThread>, dim3((unsigned)P), dim3(kPassThreads), 0, st,
                     values, n, chunk, k, partial, state, out_values, ids);
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
