// Library-wide C-ABI pieces: version and the thread-local error message.
#include "common.hpp"

namespace qasr {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(QASR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  }
  return QASR_OK;
}

}  // namespace qasr

extern "C" int qasr_version(void) { return (0 << 16) | (1 << 8) | 0; }

extern "C" const char* qasr_last_error(void) { return qasr::g_last_error.c_str(); }
