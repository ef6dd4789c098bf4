// status.cpp -- error state of the C ABI (thread-local last-error message).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <string>

#include "common.hpp"

namespace csahca {
namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* msg) {
  g_last_error = msg ? msg : "";
  return code;
}

int fail_hip(hipError_t err, const char* where) {
  char buf[512];
  std::snprintf(buf, sizeof(buf), "%s: HIP error %d (%s)", where, static_cast<int>(err),
                hipGetErrorString(err));
  g_last_error = buf;
  return CSAHCA_ERR_HIP;
}

void clear_error() { g_last_error.clear(); }

}  // namespace csahca

extern "C" const char* csahca_last_error(void) { return csahca::g_last_error.c_str(); }

extern "C" int csahca_abi_version(void) { return 1; }
