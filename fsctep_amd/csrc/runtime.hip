// Error state and library metadata of the C ABI.
#include "common.h"

#include <mutex>

namespace fsc {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(err));
    return 1;
  }
  return 0;
}

}  // namespace fsc

extern "C" {

const char* fsc_last_error(void) { return fsc::g_last_error.c_str(); }

int fsc_abi_version(void) { return 1; }

}  // extern "C"
