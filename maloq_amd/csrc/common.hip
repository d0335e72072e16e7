// Error bookkeeping for the C ABI.
#include <stdarg.h>

#include "common.h"
#include "../../include/maloq_hip.h"

namespace maloq {

static thread_local char g_err[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return MALOQ_EHIP;
  }
  return MALOQ_OK;
}

}  // namespace maloq

extern "C" const char* maloq_last_error(void) { return maloq::g_err; }

extern "C" int maloq_abi_version(void) { return MALOQ_ABI_VERSION; }
