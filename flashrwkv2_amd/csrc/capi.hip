// Library-level C ABI helpers: version, status text, last HIP error.
#include "common.h"
#include "../../include/flashrwkv2_amd.h"

namespace {
thread_local const char* g_last_error = "";
}

namespace fr2 {
void set_last_error(const char* text) { g_last_error = text; }

int record_launch() {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return FR2_OK;
  g_last_error = hipGetErrorString(e);
  return FR2_ERR_LAUNCH;
}
}  // namespace fr2

extern "C" int fr2_abi_version(void) { return 200; }

extern "C" const char* fr2_status_string(int status) {
  switch (status) {
    case FR2_OK: return "ok";
    case FR2_ERR_INVALID_ARGUMENT: return "invalid argument";
    case FR2_ERR_UNSUPPORTED: return "unsupported configuration";
    case FR2_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

// read and clear: a text reported once cannot be mistaken later for the
// cause of another failure
extern "C" const char* fr2_last_error(void) {
  const char* text = g_last_error;
  g_last_error = "";
  return text;
}
