// Library-wide C-ABI plumbing: version, thread-local error string, launch check.
#include <string>

#include "q6moe_api.h"

namespace q6moe {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(err));
    return Q6MOE_ERR_HIP;
  }
  return Q6MOE_OK;
}

}  // namespace q6moe

extern "C" int q6moe_version(void) { return 100; }

extern "C" const char* q6moe_last_error(void) { return q6moe::g_last_error.c_str(); }
