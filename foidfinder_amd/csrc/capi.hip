// ABI version and the thread-local error channel of the C ABI.
#include "common.h"

namespace ff {

static thread_local std::string g_error;

void set_error(const std::string& msg) { g_error = msg; }
void clear_error() { g_error.clear(); }

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FF_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return FF_OK;
}

}  // namespace ff

extern "C" int ff_abi_version(void) { return 1; }

extern "C" const char* ff_last_error(void) { return ff::g_error.c_str(); }
