// Batched router for the grouped prefill (the reference runtime's
// native_router, grouped_s8_u4_prefill_runtime.cpp:1085-1101): router logits
// for every token with one f32 GEMM, then the per-token top-k selection of
// aima_router_topk.
//
// logits[T][E] = X[T][H] . W[E][H]^T in f32 (2 T E H flops: 2.1 GFLOP at
// T = 2048, E = 256, H = 2048) on the f32 matrix cores
// (v_mfma_f32_32x32x2_f32: f32 operands, f32 accumulation).  A block of 8
// waves owns a 64-token x 64-expert tile; wave w computes the 32 x 32
// quarter w % 4 over the K half w / 4, and the two K halves are added
// through LDS (half 0 + half 1, the same order every call).  Each lane
// loads 4 consecutive k of its token row and of its expert row with one
// 16-byte load per 8 k: MFMA j of the 4 per step then sees k0 + 4 h + j in
// lane half h, for both operands, so the 8 k of a step are each summed once.
// An f16 input is first widened to f32 in the caller's workspace.
#include "common.h"

namespace aima {

int router_topk_launch(const float* logits, int64_t tokens, int experts, int k,
                       float min_weight_sum, int32_t* ids, float* weights, hipStream_t st,
                       float* probs);

namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kRgThreads = 512;
constexpr int kRgTile = 64;  // tokens and experts per block

__global__ __launch_bounds__(256) void widen_f16_kernel(const uint16_t* __restrict__ in,
                                                        float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = h2f(in[i]);
}

// Rows past T (tokens) or E (experts) load the last row (valid memory) and
// are never stored.  H % 16 == 0 and both matrices 16-byte aligned (checked
// on the host).
__global__ __launch_bounds__(kRgThreads) void router_gemm_kernel(
    const float* __restrict__ x, const float* __restrict__ w, int64_t T, int E, int H,
    float* __restrict__ logits) {
  __shared__ float part[4][16][64];  // K-half 1 partial sums, [quarter][acc][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = wave & 3, kh = wave >> 2;
  const int64_t t0 = (int64_t)blockIdx.x * kRgTile + 32 * (q >> 1);
  const int e0 = (int)blockIdx.y * kRgTile + 32 * (q & 1);
  const int64_t tr = t0 + (lane & 31) < T ? t0 + (lane & 31) : T - 1;
  const int er = e0 + (lane & 31) < E ? e0 + (lane & 31) : E - 1;
  const int half = H / 2;
  const float* xp = x + tr * H + kh * half + 4 * (lane >> 5);
  const float* wp = w + (int64_t)er * H + kh * half + 4 * (lane >> 5);
  f32x16_t acc = f32x16_t{};
  for (int k = 0; k < half; k += 8) {
    const float4 a = *reinterpret_cast<const float4*>(xp + k);
    const float4 b = *reinterpret_cast<const float4*>(wp + k);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
  }
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) part[q][i][lane] = acc[i];
  }
  __syncthreads();
  if (kh == 1) return;
  // lane l holds expert e0 + l % 32 of token rows 8 (i / 4) + 4 (l / 32) + i % 4
  const int e = e0 + (lane & 31);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t t = t0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    const float v = acc[i] + part[q][i][lane];
    if (t < T && e < E) logits[t * E + e] = v;
  }
}

size_t router_ws_bytes(int64_t tokens, int64_t hidden, int input_f32) {
  return input_f32 ? 0 : kWsHeader + round_up((size_t)tokens * hidden * 4, 256);
}

}  // namespace
}  // namespace aima

using namespace aima;

extern "C" int aima_router_gemm_workspace_size(int64_t tokens, int64_t hidden, int32_t input_f32,
                                               size_t* bytes) {
  AIMA_REQUIRE(bytes, "router_gemm_workspace_size: null pointer");
  AIMA_REQUIRE(tokens > 0 && hidden > 0, "router_gemm_workspace_size: sizes must be positive");
  *bytes = router_ws_bytes(tokens, hidden, input_f32);
  return AIMA_OK;
}

extern "C" int aima_router_gemm_topk(const void* hidden_states, int32_t input_f32, int64_t tokens,
                                     int64_t hidden, const float* router_weight, int32_t experts,
                                     int32_t k, float min_weight_sum, float* logits, int32_t* ids,
                                     float* weights, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  AIMA_REQUIRE(hidden_states && router_weight && logits && ids && weights,
               "router_gemm_topk: null pointer");
  AIMA_REQUIRE(tokens > 0 && hidden > 0 && tokens <= (1 << 24) && hidden <= (1 << 20),
               "router_gemm_topk: tokens must be in [1, 2^24] and hidden in [1, 2^20]");
  AIMA_REQUIRE(hidden % 16 == 0, "router_gemm_topk: hidden must be a multiple of 16");
  AIMA_REQUIRE(aligned(hidden_states, 16) && aligned(router_weight, 16),
               "router_gemm_topk: hidden_states and router_weight must be 16-byte aligned");
  AIMA_REQUIRE(experts > 0 && experts <= 1024, "router_gemm_topk: experts must be in [1, 1024]");
  AIMA_REQUIRE(k > 0 && k <= 16 && k <= experts,
               "router_gemm_topk: k must be in [1, min(16, experts)]");
  AIMA_REQUIRE(min_weight_sum > 0.f, "router_gemm_topk: minimum weight sum must be positive");
  const hipStream_t st = (hipStream_t)stream;
  const float* x = static_cast<const float*>(hidden_states);
  if (!input_f32) {
    AIMA_REQUIRE(workspace && aligned(workspace, 256) &&
                     workspace_bytes >= router_ws_bytes(tokens, hidden, 0),
                 "router_gemm_topk: an f16 input needs the workspace");
    float* wide = reinterpret_cast<float*>(static_cast<char*>(workspace) + kWsHeader);
    const int64_t n = tokens * hidden;
    hipLaunchKernelGGL(widen_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(hidden_states), wide, n);
    const int rc = launch_check("router_gemm widen");
    if (rc != AIMA_OK) return rc;
    x = wide;
  }
  {
    const dim3 grid((unsigned)((tokens + kRgTile - 1) / kRgTile),
                    (unsigned)((experts + kRgTile - 1) / kRgTile));
    hipLaunchKernelGGL(router_gemm_kernel, grid, dim3(kRgThreads), 0, st, x, router_weight,
                       tokens, experts, (int)hidden, logits);
    const int rc = launch_check("router_gemm");
    if (rc != AIMA_OK) return rc;
  }
  return router_topk_launch(logits, tokens, experts, k, min_weight_sum, ids, weights, st,
                            nullptr);
}
