// Error state and small ABI helpers shared by every entry point.
#include "common.h"

#include <string>

namespace aima {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return AIMA_OK;
  return fail(AIMA_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int launch_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return AIMA_OK;
  return fail(AIMA_E_HIP, std::string(what) + " launch failed: " + hipGetErrorString(e));
}

}  // namespace aima

extern "C" const char* aima_last_error(void) { return aima::g_last_error.c_str(); }

extern "C" int aima_version(void) { return 102; }

extern "C" int aima_workspace_error(void* workspace, uint32_t* error_bits, void* stream) {
  AIMA_REQUIRE(workspace && error_bits, "workspace_error: null pointer");
  hipStream_t st = (hipStream_t)stream;
  uint32_t v = 0;
  AIMA_HIP(hipMemcpyAsync(&v, workspace, sizeof(v), hipMemcpyDeviceToHost, st));
  AIMA_HIP(hipStreamSynchronize(st));
  const uint32_t zero = 0;
  AIMA_HIP(hipMemcpyAsync(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice, st));
  AIMA_HIP(hipStreamSynchronize(st));
  *error_bits = v;
  return AIMA_OK;
}
