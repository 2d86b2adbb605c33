// C-ABI plumbing shared by the router and grouped-GEMM entry points: the
// thread-local error message and the post-launch check.
#include "common.h"

namespace moe {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MOE_EHIP, std::string(what) + " launch failed: " + hipGetErrorString(e));
  return MOE_OK;
}

}  // namespace moe

extern "C" const char* moe_last_error(void) { return moe::g_last_error.c_str(); }

extern "C" int moe_version(void) { return 100; }
