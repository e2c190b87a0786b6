// Thread-local error reporting for the C ABI.
#include <string>

#include "common.h"

namespace ffmoe {

static thread_local std::string g_last_error;

int set_error(const std::string& msg) {
  g_last_error = msg;
  return 1;
}

int clear_error() {
  g_last_error.clear();
  return 0;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(std::string(what) + ": " + hipGetErrorString(e));
  return 0;
}

}  // namespace ffmoe

extern "C" const char* ffmoe_last_error(void) { return ffmoe::g_last_error.c_str(); }

extern "C" int ffmoe_version(void) { return 1; }
