// Batched router for the grouped prefill (the reference runtime's
// native_router, grouped_s8_u4_prefill_runtime.cpp:1085-1101): router logits
// for every token with one f32 GEMM, then the per-token top-k selection of
// aima_router_topk.
//
// logits[T][E] = X[T][H] . W[E][H]^T is a plain f32 GEMM (2 T E H flops:
// 2.1 GFLOP at T = 2048, E = 256, H = 2048), so it goes to rocBLAS
// (rocblas_sgemm, full f32) on the caller's stream; the selection is our own
// kernel.  An f16 input is first widened to f32 in the caller's workspace.
#include "common.h"

#include <rocblas/rocblas.h>

#include <mutex>
#include <unordered_map>

namespace aima {

int router_topk_launch(const float* logits, int64_t tokens, int experts, int k,
                       float min_weight_sum, int32_t* ids, float* weights, hipStream_t st,
                       float* probs);

namespace {

// One rocBLAS handle per device, created on first use; calls are
// serialized because the handle carries the stream.
std::mutex g_mu;
std::unordered_map<int, rocblas_handle> g_handles;

int rocblas_fail(rocblas_status s, const char* what) {
  return fail(AIMA_E_HIP, std::string(what) + ": " + rocblas_status_to_string(s));
}

__global__ __launch_bounds__(256) void widen_f16_kernel(const uint16_t* __restrict__ in,
                                                        float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = h2f(in[i]);
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
  AIMA_REQUIRE(tokens > 0 && hidden > 0 && tokens <= INT32_MAX && hidden <= INT32_MAX,
               "router_gemm_topk: token and hidden counts must be in [1, 2^31)");
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
    std::lock_guard<std::mutex> lock(g_mu);
    int dev = 0;
    AIMA_HIP(hipGetDevice(&dev));
    rocblas_handle h = nullptr;
    auto it = g_handles.find(dev);
    if (it == g_handles.end()) {
      const rocblas_status s = rocblas_create_handle(&h);
      if (s != rocblas_status_success) return rocblas_fail(s, "router_gemm: rocblas_create_handle");
      g_handles.emplace(dev, h);
    } else {
      h = it->second;
    }
    rocblas_status s = rocblas_set_stream(h, st);
    if (s != rocblas_status_success) return rocblas_fail(s, "router_gemm: rocblas_set_stream");
    // column-major: logits (E x T, ld E) = W^T (W: H x E, ld H)^T . X (H x T, ld H)
    const float one = 1.f, zero = 0.f;
    s = rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none, experts,
                      (rocblas_int)tokens, (rocblas_int)hidden, &one, router_weight,
                      (rocblas_int)hidden, x, (rocblas_int)hidden, &zero, logits, experts);
    if (s != rocblas_status_success) return rocblas_fail(s, "router_gemm: rocblas_sgemm");
  }
  return router_topk_launch(logits, tokens, experts, k, min_weight_sum, ids, weights, st,
                            nullptr);
}
