// Error text and version of the C-ABI (include/vllm_mi355x.h).
#include "common.h"

#include "../../include/vllm_mi355x.h"

namespace vq {
namespace {
thread_local std::string g_error;
}  // namespace

int fail(const std::string& message) {
  g_error = message;
  return kInvalidArgument;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    g_error = std::string(what) + ": " + hipGetErrorString(err);
    return kHipFailure;
  }
  return kOk;
}

}  // namespace vq

extern "C" const char* vllm_mi355x_last_error(void) { return vq::g_error.c_str(); }
extern "C" int vllm_mi355x_abi_version(void) { return VLLM_MI355X_ABI_VERSION; }
