// C-ABI plumbing shared by all entry points: thread-local error message, launch checks and
// library constants.
#include <stdarg.h>

#include "gs_host.h"

namespace gs {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return GS_ERR_LAUNCH;
  }
  return GS_OK;
}

}  // namespace gs

extern "C" const char* gs_last_error(void) { return gs::g_last_error; }
extern "C" int gs_version(void) { return 1; }
extern "C" int gs_splat_record_floats(void) { return gs::kRecFloats; }
extern "C" int gs_grad2d_floats(void) { return gs::kGrad2D; }
