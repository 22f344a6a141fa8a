// Error state and version query of the C ABI (include/my_vllm_amd.h).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "mva_capi.h"

namespace mva {
namespace {
thread_local char g_last_error[512] = "";
}

int set_error(const char* msg) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return -1;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return 0;
  std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(err));
  return -2;
}

}  // namespace mva

extern "C" const char* mva_last_error(void) { return mva::g_last_error; }

extern "C" int mva_abi_version(void) { return 11; }
