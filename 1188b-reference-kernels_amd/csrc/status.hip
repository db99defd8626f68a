// Status codes, the per-thread last-error message and launch checking.
#include <stdarg.h>
#include <stdio.h>

#include "moe_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace moe {

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(MOE_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return MOE_OK;
}

}  // namespace moe

extern "C" {

int moe_abi_version(void) { return MOE_DISPATCH_ABI_VERSION; }

const char *moe_status_string(int status) {
  switch (status) {
    case MOE_OK: return "ok";
    case MOE_ERR_INVALID_ARG: return "invalid argument";
    case MOE_ERR_SHAPE: return "bad shape";
    case MOE_ERR_ALIGN: return "misaligned pointer";
    case MOE_ERR_CAPACITY: return "size beyond supported capacity";
    case MOE_ERR_WORKSPACE: return "workspace missing or too small";
    case MOE_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

const char *moe_last_error(void) { return g_last_error; }

}  // extern "C"
