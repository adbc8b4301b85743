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

// An error left pending by earlier, unrelated HIP calls is taken off the error slot on entry
// (so it is not blamed on this call) and reported alongside any failure of this call.
static thread_local hipError_t g_stale = hipSuccess;

void clear_error() {
  g_last_error[0] = 0;
  g_stale = hipGetLastError();
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    if (g_stale != hipSuccess) {
      set_error("%s: %s (an earlier HIP call had left: %s)", what, hipGetErrorString(e),
                hipGetErrorString(g_stale));
    } else {
      set_error("%s: %s", what, hipGetErrorString(e));
    }
    return GS_ERR_LAUNCH;
  }
  return GS_OK;
}

}  // namespace gs

extern "C" const char* gs_last_error(void) { return gs::g_last_error; }
extern "C" int gs_version(void) { return 1; }
extern "C" int gs_splat_record_floats(void) { return gs::kRecFloats; }
extern "C" int gs_grad2d_floats(void) { return gs::kGrad2D; }
