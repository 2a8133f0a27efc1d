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
// logits followed by this selection -- at K = 2048 in one launch
// (lm_head_topk_kernel): the selection blocks follow the matvec blocks in
// the grid and read value-tagged copies of the logits, so the selection
// starts while the matvec's last blocks still run, with no launch gap.  A
// variant with the reference's shape -- every matvec block writing its own
// partial top-k, the selection then running over those candidates --
// measured slower: the block barrier and ranking in each of the 7,760
// matvec blocks cost 5.6 us at N = 248,320, while the selection is bound by
// latency, not by the 1 MB of logits it reads.
#include "common.h"
#include "matvec_block.h"

#include <math.h>
#include <stdlib.h>

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
constexpr int kMaxCand = 256;  // survivors one wave selects from (4 per lane)

// The selection's launch counter, kept in the workspace header at byte 132
// (the error word is at 0; bytes 128..131 stay zero): any start value, and
// it advances by one per launch.  A launch tags both words of each of its
// picks with the full 32-bit counter value (see pick_high_word), so a slot
// is taken only when it was written by this launch: a zero-filled slot, a
// slot of an earlier launch and data other entry points left in the same
// memory all fail the check (short of matching two 32-bit tags at once).
constexpr size_t kTopkLaunchOffset = 132;

// Each (value, index) pair as one 64-bit key: a larger key is the better
// pair (larger value, then lower index), so every ordering test is a single
// unsigned compare.  High word: the value's bits made monotone (sign set: all
// bits flipped; otherwise the sign bit set), -0 and +0 alike (equal values);
// low word: (0x7fffffff - index) << 1, bit 0 set for a -0 value so the value
// decodes bit for bit.  NaN and the empty pair are key 0, below every number
// (the smallest, -inf, has high word 0x007fffff).  Indices are < 2^31.
__device__ __forceinline__ uint64_t pair_key(float v, int i) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const bool negzero = b == 0x80000000u;
  const uint32_t m = negzero ? 0x80000000u : (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  const uint32_t lo = ((uint32_t)(0x7fffffff - i) << 1) | (negzero ? 1u : 0u);
  return v != v ? 0ull : ((uint64_t)m << 32) | lo;
}
__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t m = (uint32_t)(key >> 32);
  const uint32_t b = (key & 1u) ? 0x80000000u : (m & 0x80000000u) ? (m & 0x7fffffffu) : ~m;
  return key == 0 ? -INFINITY : __builtin_bit_cast(float, b);
}
__device__ __forceinline__ int key_index(uint64_t key) {
  return key == 0 ? kNoIndex : 0x7fffffff - (int)((uint32_t)key >> 1);
}

__device__ __forceinline__ uint64_t max_key(uint64_t a, uint64_t b) { return a > b ? a : b; }
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_key(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t read_key(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}
// The largest key of each 16-lane row, in every lane of the row: quad_perm
// [1,0,3,2] and [2,3,0,1] (the quad), row_half_mirror (the 8-lane half),
// row_mirror (the row).
__device__ __forceinline__ uint64_t row_best_key(uint64_t v) {
  v = max_key(v, dpp_key<0xB1>(v));
  v = max_key(v, dpp_key<0x4E>(v));
  v = max_key(v, dpp_key<0x141>(v));
  return max_key(v, dpp_key<0x140>(v));
}
__device__ __forceinline__ uint64_t wave_best_key(uint64_t v) {
  v = row_best_key(v);
  return max_key(max_key(read_key(v, 0), read_key(v, 16)), max_key(read_key(v, 32), read_key(v, 48)));
}

// k rounds of a wave-wide maximum over PER keys per lane: lane r < k returns
// the rank-r key (0 once the numbers run out).  Keys other than 0 are
// unique, so each round removes exactly its pick.
template <int PER>
__device__ __forceinline__ uint64_t wave_topk_keys(uint64_t (&c)[PER], int k) {
  const int lane = threadIdx.x & 63;
  uint64_t res = 0;
  for (int r = 0; r < k; ++r) {
    uint64_t b = c[0];
#pragma unroll
    for (int j = 1; j < PER; ++j) b = max_key(b, c[j]);
    b = wave_best_key(b);
    res = lane == r ? b : res;
#pragma unroll
    for (int j = 0; j < PER; ++j) c[j] = c[j] == b ? 0ull : c[j];
  }
  return res;
}

struct alignas(16) Key2 {
  uint64_t a, b;
};

struct SelectLds {
  alignas(16) uint64_t rb[kRowBests];         // row bests
  alignas(16) uint64_t cand[kMaxCand];        // survivors
  alignas(16) uint64_t wl[kWaves * kTopkMax]; // ranked picks / per-wave lists
  int count;
};

// The block's top-k keys of PER keys per thread: wave 0 lane r < k returns
// the rank-r key (0: fewer than r + 1 numbers); every other thread returns
// 0.  Every thread of the block calls it.
//
// Threshold filter first: every 16-lane row finds its best key (DPP inside
// the row); the k-th best of the 16 row bests, T, bounds the block's top-k
// from below (the k row bests at or above T are k keys at least as good),
// so only keys at or above T can be picked.  Each lane counts its keys at or
// above T, takes that many slots with one LDS atomic add and writes them
// (their order does not matter).  Up to 64 survivors (the usual case: about
// the 16 row bests): lane l ranks survivor l against all of them and the
// survivor of rank r < k is pick r.  Up to 256: wave 0 selects by k rounds of
// a wave-wide maximum.  More (a chunk whose best values crowd into few rows):
// every wave selects its own k and wave 0 selects from the 4 lists.
template <int PER>
__device__ uint64_t block_select(const uint64_t (&key)[PER], int k, SelectLds& S) {
  static_assert((PER & (PER - 1)) == 0, "PER is a power of two");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // the lane's best by a pairwise tree (independent compares at each level),
  // then the row's best
  uint64_t t[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) t[j] = key[j];
#pragma unroll
  for (int w = PER / 2; w > 0; w /= 2) {
#pragma unroll
    for (int j = 0; j < w; ++j) t[j] = max_key(t[j], t[j + w]);
  }
  const uint64_t rbest = row_best_key(t[0]);
  if ((lane & 15) == 0) S.rb[wave * 4 + (lane >> 4)] = rbest;
  if (threadIdx.x == 0) S.count = 0;
  __syncthreads();
  // T = the rank-(k-1) row best, found by every wave (row bests other than 0
  // are unique; with fewer than k of them there is no filter: T stays 1,
  // below every number's key)
  uint64_t T = 1;
  {
    const uint64_t mine = S.rb[lane & (kRowBests - 1)];
    int rank = 0;
#pragma unroll
    for (int w = 0; w < kRowBests; w += 2) {
      const Key2 a = *reinterpret_cast<const Key2*>(&S.rb[w]);
      rank += (a.a > mine ? 1 : 0) + (a.b > mine ? 1 : 0);
    }
    const uint64_t hit = __ballot(lane < kRowBests && rank == k - 1 && mine != 0);
    if (hit) T = read_key(mine, (int)__builtin_ctzll(hit));
  }
  int c = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) c += key[j] >= T ? 1 : 0;
  int slot = 0;
  if (c) slot = atomicAdd(&S.count, c);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (key[j] >= T) {
      if (slot < kMaxCand) S.cand[slot] = key[j];
      ++slot;
    }
  }
  __syncthreads();
  const int total = S.count;
  if (total <= kMaxCand) {
    if (wave != 0) return 0;
    if (total <= 64) {
      const uint64_t mine = lane < total ? S.cand[lane] : 0;
      // survivors padded with 0 keys to a multiple of 16, then compared 16
      // at a time from eight 16-byte LDS reads (every lane reads the same
      // words), so the reads are in flight together
      const int tot16 = (total + 15) & ~15;
      if (lane >= total && lane < tot16) S.cand[lane] = 0;
      wave_lds_sync();
      int rank = 0;
      for (int j = 0; j < tot16; j += 16) {
        Key2 a[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] = *reinterpret_cast<const Key2*>(&S.cand[j + 2 * u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) rank += (a[u].a > mine ? 1 : 0) + (a[u].b > mine ? 1 : 0);
      }
      if (lane < total && rank < k) S.wl[rank] = mine;
      if (lane >= total && lane < k) S.wl[lane] = 0;  // fewer than k numbers
      wave_lds_sync();
      return lane < k ? S.wl[lane] : 0;
    }
    uint64_t c4[kMaxCand / 64];
#pragma unroll
    for (int j = 0; j < kMaxCand / 64; ++j) {
      const int q = lane + 64 * j;
      c4[j] = q < total ? S.cand[q] : 0;
    }
    return wave_topk_keys<kMaxCand / 64>(c4, k);
  }
  uint64_t own[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) own[j] = key[j];
  const uint64_t wv = wave_topk_keys<PER>(own, k);
  if (lane < k) S.wl[wave * k + lane] = wv;
  __syncthreads();
  if (wave != 0) return 0;
  uint64_t m1[1] = {lane < kWaves * k ? S.wl[lane] : 0ull};
  return wave_topk_keys<1>(m1, k);
}

// A partial pick (a key) as two 64-bit words, each stored and loaded whole:
// the key's high word with the launch number, and its low word with the
// launch number xor kTagMix.  Each word validates itself; a slot is fresh
// when both carry this launch's tags.  (kTagMix is non-zero, so an all-zero
// slot never passes, whatever the counter.)
constexpr uint32_t kTagMix = 0x5bd1e995u;
__device__ __forceinline__ uint64_t pick_high_word(uint64_t key, uint32_t launch) {
  return (key >> 32) | ((uint64_t)launch << 32);
}
__device__ __forceinline__ uint64_t pick_low_word(uint64_t key, uint32_t launch) {
  return (key & 0xffffffffull) | ((uint64_t)(launch ^ kTagMix) << 32);
}
constexpr uint32_t kSpinLimit = 1u << 22;

// The final selection over the P * k = np picks, FPER per thread: block 0
// reads every slot (device-scope loads, both words whole) until each word
// carries this launch's tag -- a spin limit sets AIMA_DEVERR_TIMEOUT in the
// error word -- then selects from the keys.  Instantiated per FPER so only
// FPER keys (and their loads in flight) occupy registers.
template <int FPER>
__device__ __forceinline__ void merge_partials(const uint64_t* __restrict__ partial, int np, int k,
                                               uint32_t launch, uint32_t* __restrict__ err,
                                               SelectLds& S, float* __restrict__ out_v,
                                               int32_t* __restrict__ out_i) {
  const uint32_t tag_lo = launch ^ kTagMix;
  uint64_t key[FPER];
  for (uint32_t spins = 0;; ++spins) {
    bool fresh = true;
#pragma unroll
    for (int j = 0; j < FPER; ++j) {
      const int q = (int)threadIdx.x + kPassThreads * j;
      const int qc = q < np ? q : np - 1;
      const uint64_t wh =
          __hip_atomic_load(&partial[2 * qc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint64_t wl =
          __hip_atomic_load(&partial[2 * qc + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      fresh = fresh && (uint32_t)(wh >> 32) == launch && (uint32_t)(wl >> 32) == tag_lo;
      key[j] = q < np ? (wh << 32) | (wl & 0xffffffffull) : 0ull;
    }
    if (__syncthreads_and(fresh)) break;
    if (spins > kSpinLimit) {
      if (threadIdx.x == 0) atomicOr(err, AIMA_DEVERR_TIMEOUT);
      break;
    }
  }
  const uint64_t r = block_select<FPER>(key, k, S);
  if ((int)threadIdx.x < k) {
    out_v[threadIdx.x] = key_value(r);
    out_i[threadIdx.x] = key_index(r);
  }
}

// The selection's second half, shared by topk_kernel and the LM head's fused
// kernel: selection block b of P holds its chunk's keys and selects the
// chunk's k best; with P = 1 those are the result.  Otherwise every block
// stores its picks tagged with the launch number it read (device-scope
// stores); block 0 then reads all P * k slots (device-scope loads) until
// every word carries this launch's tag, selects the final k and advances
// the counter.  No block waits for its own stores, takes a ticket or writes
// back or invalidates a cache (a __threadfence per block made the selection
// take 70 us instead of a few; a ticket counter costs every block a store
// and an atomic round trip).  All P <= 256 selection blocks become resident,
// so block 0's wait ends.  MAXF bounds the picks per thread of the merge
// (P * k <= 256 * MAXF).
template <int PER, int MAXF>
__device__ void select_and_merge(const uint64_t (&key)[PER], int k, int P, int b,
                                 uint32_t launch, uint64_t* __restrict__ partial,
                                 uint32_t* __restrict__ state, float* __restrict__ out_v,
                                 int32_t* __restrict__ out_i) {
  __shared__ SelectLds S;
  uint32_t* const err = state;  // the workspace error word (byte 0)
  uint32_t* const epoch_word = state + kTopkLaunchOffset / 4;
  const uint64_t r = block_select<PER>(key, k, S);
  if (P == 1) {
    if ((int)threadIdx.x < k) {
      out_v[threadIdx.x] = key_value(r);
      out_i[threadIdx.x] = key_index(r);
    }
    return;
  }
  if ((int)threadIdx.x < k) {  // wave 0 holds the picks
    uint64_t* slot = partial + 2 * ((int64_t)b * k + threadIdx.x);
    __hip_atomic_store(slot, pick_high_word(r, launch), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(slot + 1, pick_low_word(r, launch), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  if (b != 0) return;
  const int np = P * k;  // <= 256 * 16 = 4096
  if (MAXF <= 2 || np <= 2 * kPassThreads) {
    merge_partials<2>(partial, np, k, launch, err, S, out_v, out_i);
  } else if (MAXF <= 4 || np <= 4 * kPassThreads) {
    merge_partials<4>(partial, np, k, launch, err, S, out_v, out_i);
  } else if (MAXF <= 8 || np <= 8 * kPassThreads) {
    merge_partials<8>(partial, np, k, launch, err, S, out_v, out_i);
  } else {
    merge_partials<16>(partial, np, k, launch, err, S, out_v, out_i);
  }
  // device scope, like the loads that read it: the next launch's blocks
  // (on any XCD) must see the new counter, never this launch's
  if (threadIdx.x == 0) {
    __hip_atomic_store(epoch_word, launch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The selection over a values array (see the file comment): block b owns
// values [b * chunk, min(n, (b + 1) * chunk)).
template <int PER>
__global__ __launch_bounds__(kPassThreads) void topk_kernel(
    const float* __restrict__ vals, int64_t n, int64_t chunk, int k, uint64_t* __restrict__ partial,
    uint32_t* __restrict__ state, float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  const int64_t base = (int64_t)blockIdx.x * chunk;
  const int64_t end = base + chunk < n ? base + chunk : n;
  uint32_t launch = 0;
  if (gridDim.x > 1) {
    launch = __hip_atomic_load(state + kTopkLaunchOffset / 4, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  }
  uint64_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    // positions past the chunk read its last element (straight-line loads,
    // all in flight at once) and are then emptied
    const int64_t p = base + threadIdx.x + (int64_t)kPassThreads * j;
    const int64_t pc = p < end ? p : end - 1;
    const float val = vals[pc];
    key[j] = p < end ? pair_key(val, (int)p) : 0ull;
  }
  select_and_merge<PER, 16>(key, k, (int)gridDim.x, (int)blockIdx.x, launch, partial, state,
                            out_v, out_i);
}

// The fused kernel's selection takes 8 values per thread (chunks of 2,048)
// and its merge at most 4 picks per thread (P * k <= 1,024), so it holds
// fewer registers than topk_kernel (16 of each): the kernel's register count
// sets the occupancy of its matvec blocks too.
constexpr int kFusedPer = 8;
constexpr int kFusedMergePer = 4;

// U4 LM head with top-k in one launch: blocks 0 .. nmv - 1 are the matvec's
// (K = 2048, RG row passes per wave), each also storing its logits tagged;
// blocks nmv .. nmv + P - 1 are the selection's.  The hardware dispatches
// blocks in order, so the selection blocks start only once every matvec
// block has been dispatched -- they run beside the matvec's tail -- and no
// matvec block ever waits for them (were dispatch out of order, the at most
// 256 waiting selection blocks would still leave most of the chip's block
// slots to the matvec).  Selection block b reads the tagged logits of its
// chunk (device-scope loads, a short sleep between rounds) until all carry
// this launch's tag, then selects as topk_kernel's blocks do.  Every block
// reads the launch counter first; the counter advances only after the
// selection has seen every matvec block's logits, so all blocks of a launch
// read one value.
template <int RG>
__global__ __launch_bounds__(kPassThreads) void lm_head_topk_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ qw,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zp, int64_t n,
    int group_log2, float* __restrict__ logits, int nmv, int64_t chunk, int k,
    uint64_t* __restrict__ tagged, uint64_t* __restrict__ partial, uint32_t* __restrict__ state,
    float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  const uint32_t launch = __hip_atomic_load(state + kTopkLaunchOffset / 4, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
  if ((int)blockIdx.x < nmv) {
    matvec_block<64, RG>(x, qw, scale, zp, n, group_log2, logits, 1, blockIdx.x, tagged, launch);
    return;
  }
  const int b = (int)blockIdx.x - nmv;
  const int P = (int)gridDim.x - nmv;
  const int64_t base = (int64_t)b * chunk;
  const int64_t end = base + chunk < n ? base + chunk : n;
  uint64_t key[kFusedPer];
  for (uint32_t spins = 0;; ++spins) {
    bool fresh = true;
#pragma unroll
    for (int j = 0; j < kFusedPer; ++j) {
      const int64_t p = base + threadIdx.x + (int64_t)kPassThreads * j;
      const int64_t pc = p < end ? p : end - 1;
      const uint64_t w = __hip_atomic_load(&tagged[pc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t bits = (uint32_t)w;
      fresh = fresh && (uint32_t)(w >> 32) == logit_tag(bits, launch);
      key[j] = p < end ? pair_key(__builtin_bit_cast(float, bits), (int)p) : 0ull;
    }
    if (__syncthreads_and(fresh)) break;
    if (spins > kSpinLimit) {
      if (threadIdx.x == 0) atomicOr(state, AIMA_DEVERR_TIMEOUT);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  select_and_merge<kFusedPer, kFusedMergePer>(key, k, P, b, launch, partial, state, out_v,
                                              out_i);
  // one selection block: no merge advanced the counter, this block does (it
  // has seen every matvec block's logits, so all of them have read it)
  if (P == 1 && threadIdx.x == 0) {
    __hip_atomic_store(state + kTopkLaunchOffset / 4, launch + 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

int partial_blocks(int64_t n) {
  const int64_t p = (n + kChunkMax - 1) / kChunkMax;
  return (int)(p < kMaxPartials ? p : kMaxPartials);
}

// The fused LM head's selection blocks: chunks of at most 2,048 values.
constexpr int64_t kFusedChunkMax = (int64_t)kPassThreads * kFusedPer;
int fused_blocks(int64_t n) {
  const int64_t p = (n + kFusedChunkMax - 1) / kFusedChunkMax;
  return (int)(p < kMaxPartials ? p : kMaxPartials);
}
bool fused_fits(int64_t n, int k) {
  return n <= kFusedChunkMax * kMaxPartials && fused_blocks(n) * k <= kFusedMergePer * kPassThreads;
}

// Workspace: the header (error word at 0, launch counter at
// kTopkLaunchOffset), the LM head's tagged logits (8 bytes per value; unused
// by aima_topk_f32), then the P * k partial picks, 16 bytes each.
size_t tagged_bytes(int64_t n) { return round_up((size_t)n * 8, 256); }
size_t topk_ws_bytes(int64_t n, int k) {
  return kWsHeader + tagged_bytes(n) + round_up((size_t)fused_blocks(n) * k * 16, 256);
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
    partial = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsHeader + tagged_bytes(n));
  }
  hipLaunchKernelGGL(topk_kernel<kPerThread>, dim3((unsigned)P), dim3(kPassThreads), 0, st,
                     values, n, chunk, k, partial, state, out_values, ids);
  return launch_check("topk");
}

// The LM head in one launch (K = 2048): lm_head_topk_kernel with the
// matvec's row-group rule (8 row passes per wave once that leaves >= 512
// blocks, else 4).
int lm_head_fused_launch(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                         const uint8_t* zp, int64_t n, int glog2, float* logits, int k,
                         int32_t* ids, float* out_values, void* ws, hipStream_t st) {
  const int P = fused_blocks(n);
  const int64_t chunk = (n + P - 1) / P;
  uint32_t* state = static_cast<uint32_t*>(ws);
  uint64_t* tagged = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsHeader);
  uint64_t* partial =
      reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsHeader + tagged_bytes(n));
  const int64_t rows8 = 4 * 8;
  if ((n + rows8 - 1) / rows8 >= 512) {
    const int nmv = (int)((n + rows8 - 1) / rows8);
    hipLaunchKernelGGL(lm_head_topk_kernel<8>, dim3((unsigned)(nmv + P)), dim3(kPassThreads), 0,
                       st, x, qw, scale, zp, n, glog2, logits, nmv, chunk, k, tagged, partial,
                       state, out_values, ids);
  } else {
    const int64_t rows4 = 4 * 4;
    const int nmv = (int)((n + rows4 - 1) / rows4);
    hipLaunchKernelGGL(lm_head_topk_kernel<4>, dim3((unsigned)(nmv + P)), dim3(kPassThreads), 0,
                       st, x, qw, scale, zp, n, glog2, logits, nmv, chunk, k, tagged, partial,
                       state, out_values, ids);
  }
  return launch_check("lm_head_topk");
}

// AIMA_LM_HEAD_FUSED=0 selects the two-launch LM head (matvec, then
// topk_kernel) everywhere; read once per process.
bool lm_head_fused_enabled() {
  static const bool on = [] {
    const char* e = getenv("AIMA_LM_HEAD_FUSED");
    return !(e && e[0] == '0');
  }();
  return on;
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
  if (k == 2048 && lm_head_fused_enabled() && workspace && aligned(workspace, 256) &&
      workspace_bytes >= topk_ws_bytes(n, topk) && fused_fits(n, topk)) {
    return lm_head_fused_launch(x, qweight, scale, zp, n, glog2, logits, topk, ids, values,
                                workspace, st);
  }
  rc = u4_matvec_dispatch(x, qweight, scale, zp, n, k, glog2, logits, 1, st);
  if (rc != AIMA_OK) return rc;
  return topk_launch(logits, n, topk, ids, values, workspace, workspace_bytes, st);
}
