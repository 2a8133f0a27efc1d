// Device top-k over f32 values and the U4 LM head with top-k, for gfx950.
//
// Order: value descending, the lower index first among equal values -- the
// order of the reference's LM-head partial top-8 (q4x8_matvec.cl:973-1021:
// an insertion that keeps an earlier index ahead of an equal later value).
// NaN values never compare better than anything, so they are never chosen
// ahead of a number.
//
// Two passes.  Pass 1: P blocks of 1024 threads, block b owns a contiguous
// chunk of at most 4096 values (4 per thread) and picks its k best (a
// threshold filter, then k rounds of a wave-wide (value, index) maximum over
// the survivors; see topk_pass_kernel).  Pass 2: one block runs the same
// selection over the P * k (value, index) candidates.  P <= 256, so
// n <= 1,048,576 and the candidates of pass 2 fit one block.
#include "common.h"

#include <math.h>

namespace aima {

int u4_matvec_dispatch(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                       const uint8_t* zp, int64_t n, int64_t k, int glog2, void* y,
                       int out_f32, hipStream_t st);
int group_log2_of(int group);

namespace {

constexpr int kTopkMax = 16;
constexpr int kPassThreads = 1024;
constexpr int kPerThread = 4;
constexpr int kMaxPartials = 256;
constexpr int64_t kChunkMax = (int64_t)kPassThreads * kPerThread;
constexpr int64_t kTopkMaxN = kChunkMax * kMaxPartials;
constexpr int kNoIndex = 0x7fffffff;

__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  return av > bv || (av == bv && ai < bi);
}

// k rounds of a wave-wide maximum over PER candidates per lane; lane r ends
// holding the rank-r pick (r < k).
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

constexpr int kWaves = kPassThreads / 64;
constexpr int kMaxCand = 256;  // candidates one wave selects from (4 per lane)

// idx null: a value's index is its position.
//
// Threshold filter first: each wave finds its best (value, index) pair; the
// k-th best of the 16 wave bests, T, bounds the block's top-k from below
// (the k wave bests at or above T are k pairs at least as good), so only
// pairs at or above T can be picked.  They are compacted into LDS (ballots
// give each its slot) and wave 0 selects from them.  When ties leave more
// than kMaxCand such pairs, every wave selects its own k and wave 0 merges
// the 16 lists instead.
__global__ __launch_bounds__(kPassThreads) void topk_pass_kernel(
    const float* __restrict__ vals, const int32_t* __restrict__ idx, int64_t n, int64_t chunk,
    int k, float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  __shared__ float s_v[kWaves * kTopkMax];
  __shared__ int s_i[kWaves * kTopkMax];
  __shared__ float s_wv[kWaves];
  __shared__ int s_wi[kWaves];
  __shared__ int s_cnt[kWaves];
  __shared__ float s_cv[kMaxCand];
  __shared__ int s_ci[kMaxCand];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t base = (int64_t)blockIdx.x * chunk;
  const int64_t end = base + chunk < n ? base + chunk : n;
  float v[kPerThread];
  int ix[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t p = base + threadIdx.x + (int64_t)kPassThreads * j;
    if (p < end) {
      v[j] = vals[p];
      ix[j] = idx ? idx[p] : (int)p;
    } else {
      v[j] = -INFINITY;
      ix[j] = kNoIndex;
    }
  }
  // wave bests
  float bv = -INFINITY;
  int bi = kNoIndex;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    if (better(v[j], ix[j], bv, bi)) {
      bv = v[j];
      bi = ix[j];
    }
  }
  wave_best_pair(bv, bi);
  if (lane == 0) {
    s_wv[wave] = bv;
    s_wi[wave] = bi;
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
      mv = s_wv[lane];
      mi = s_wi[lane];
      rank = 0;
      for (int w = 0; w < kWaves; ++w) rank += better(s_wv[w], s_wi[w], mv, mi) ? 1 : 0;
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
  bool q[kPerThread];
  uint64_t mask[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    q[j] = ix[j] != kNoIndex && (better(v[j], ix[j], tv, ti) || (v[j] == tv && ix[j] == ti));
    mask[j] = __ballot(q[j]);
    cnt += __builtin_popcountll(mask[j]);
  }
  if (lane == 0) s_cnt[wave] = cnt;
  __syncthreads();
  int wbase = 0, total = 0;
  for (int w = 0; w < kWaves; ++w) {
    const int c = s_cnt[w];
    wbase += w < wave ? c : 0;
    total += c;
  }
  if (total <= kMaxCand) {
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int off = wbase;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      if (q[j]) {
        const int slot = off + __builtin_popcountll(mask[j] & below);
        s_cv[slot] = v[j];
        s_ci[slot] = ix[j];
      }
      off += __builtin_popcountll(mask[j]);
    }
    __syncthreads();
    if (wave == 0) {
      float c[kMaxCand / 64];
      int ci[kMaxCand / 64];
#pragma unroll
      for (int j = 0; j < kMaxCand / 64; ++j) {
        const int slot = lane + 64 * j;
        if (slot < total) {
          c[j] = s_cv[slot];
          ci[j] = s_ci[slot];
        } else {
          c[j] = -INFINITY;
          ci[j] = kNoIndex;
        }
      }
      float wv;
      int wi;
      wave_topk<kMaxCand / 64>(c, ci, k, wv, wi);
      if (lane < k) {
        out_v[(int64_t)blockIdx.x * k + lane] = wv;
        out_i[(int64_t)blockIdx.x * k + lane] = wi;
      }
    }
    return;
  }
  // many ties at the threshold: per-wave selection, then a merge
  float wv;
  int wi;
  wave_topk<kPerThread>(v, ix, k, wv, wi);
  if (lane < k) {
    s_v[wave * k + lane] = wv;
    s_i[wave * k + lane] = wi;
  }
  __syncthreads();
  if (wave == 0) {
    constexpr int kCandPer = kWaves * kTopkMax / 64;
    float c[kCandPer];
    int ci[kCandPer];
#pragma unroll
    for (int j = 0; j < kCandPer; ++j) {
      const int qi = lane + 64 * j;
      if (qi < kWaves * k) {
        c[j] = s_v[qi];
        ci[j] = s_i[qi];
      } else {
        c[j] = -INFINITY;
        ci[j] = kNoIndex;
      }
    }
    wave_topk<kCandPer>(c, ci, k, wv, wi);
    if (lane < k) {
      out_v[(int64_t)blockIdx.x * k + lane] = wv;
      out_i[(int64_t)blockIdx.x * k + lane] = wi;
    }
  }
}

int partial_blocks(int64_t n) {
  const int64_t p = (n + kPassThreads - 1) / kPassThreads;
  return (int)(p < kMaxPartials ? p : kMaxPartials);
}

size_t topk_ws_bytes(int64_t n, int k) {
  return 2 * round_up((size_t)partial_blocks(n) * k * 4, 256);
}

int topk_launch(const float* values, int64_t n, int k, int32_t* ids, float* out_values, void* ws,
                size_t ws_bytes, hipStream_t st) {
  const int P = partial_blocks(n);
  const int64_t chunk = (n + P - 1) / P;
  if (P == 1) {
    hipLaunchKernelGGL(topk_pass_kernel, dim3(1), dim3(kPassThreads), 0, st, values, nullptr, n,
                       chunk, k, out_values, ids);
    return launch_check("topk");
  }
  AIMA_REQUIRE(ws && ws_bytes >= topk_ws_bytes(n, k), "topk: workspace too small");
  char* p = static_cast<char*>(ws);
  float* pv = reinterpret_cast<float*>(p);
  int32_t* pi = reinterpret_cast<int32_t*>(p + round_up((size_t)P * k * 4, 256));
  hipLaunchKernelGGL(topk_pass_kernel, dim3((unsigned)P), dim3(kPassThreads), 0, st, values,
                     nullptr, n, chunk, k, pv, pi);
  hipLaunchKernelGGL(topk_pass_kernel, dim3(1), dim3(kPassThreads), 0, st, pv, pi,
                     (int64_t)P * k, (int64_t)P * k, k, out_values, ids);
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
  AIMA_REQUIRE(partial_blocks(n) == 1 || (workspace && workspace_bytes >= topk_ws_bytes(n, topk)),
               "lm_head_topk: workspace too small");
  const hipStream_t st = (hipStream_t)stream;
  rc = u4_matvec_dispatch(x, qweight, scale, zp, n, k, glog2, logits, 1, st);
  if (rc != AIMA_OK) return rc;
  return topk_launch(logits, n, topk, ids, values, workspace, workspace_bytes, st);
}
