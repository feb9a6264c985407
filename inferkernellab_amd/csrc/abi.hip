// C-ABI plumbing shared by every entry point: the thread-local error
// message and HIP launch checking.
#include "ikl_common.h"

namespace ikl {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(IKL_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return IKL_OK;
}

}  // namespace ikl

extern "C" const char *ikl_last_error(void) { return ikl::g_last_error.c_str(); }

// Build provenance, set by the build: a hash of the kernel sources and the
// header, and the git revision they were built from (+ "-dirty" when the
// working tree differed from it).
#ifndef IKL_BUILD_INFO
#define IKL_BUILD_INFO "src:unknown,git:unknown"
#endif

extern "C" const char *ikl_version(void) { return "ikl_paged 0.1 gfx950 " IKL_BUILD_INFO; }

extern "C" int32_t ikl_abi_version(void) { return IKL_ABI_VERSION; }
