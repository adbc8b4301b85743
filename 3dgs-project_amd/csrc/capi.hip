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

// Stage marks (measurement only): while enabled on a thread, the entry points record a HIP event
// on their stream at their internal stage boundaries. The events are created on first use and
// kept for the next measurement.
constexpr int kMaxMarks = 64;
static thread_local bool g_marks_on = false;
static thread_local int g_marks_n = 0;
static thread_local hipEvent_t g_marks_ev[kMaxMarks] = {};
static thread_local const char* g_marks_name[kMaxMarks] = {};

void stage_mark(const char* name, hipStream_t st) {
  if (!g_marks_on || g_marks_n >= kMaxMarks) return;
  hipEvent_t& ev = g_marks_ev[g_marks_n];
  if (!ev && hipEventCreate(&ev) != hipSuccess) {
    ev = nullptr;
    (void)hipGetLastError();
    return;
  }
  if (hipEventRecord(ev, st) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  g_marks_name[g_marks_n++] = name;
}

}  // namespace gs

extern "C" int gs_stage_marks(int enable) {
  gs::clear_error();
  gs::g_marks_on = enable != 0;
  gs::g_marks_n = 0;
  return GS_OK;
}

extern "C" int gs_stage_marks_read(float* ms, const char** names, int max) {
  gs::clear_error();
  GS_REQUIRE(max >= 0 && (max == 0 || (ms && names)), -GS_ERR_ARG, "invalid stage mark arguments");
  const int n = gs::g_marks_n < max ? gs::g_marks_n : max;
  if (n > 0 && hipEventSynchronize(gs::g_marks_ev[gs::g_marks_n - 1]) != hipSuccess) {
    gs::check_launch("stage marks");
    return -GS_ERR_LAUNCH;
  }
  for (int i = 0; i < n; ++i) {
    names[i] = gs::g_marks_name[i];
    ms[i] = 0.0f;
    if (i > 0 && hipEventElapsedTime(&ms[i], gs::g_marks_ev[i - 1], gs::g_marks_ev[i]) != hipSuccess) {
      gs::check_launch("stage marks");
      return -GS_ERR_LAUNCH;
    }
  }
  return n;
}

extern "C" const char* gs_last_error(void) { return gs::g_last_error; }
extern "C" int gs_version(void) { return 1; }
extern "C" int gs_splat_record_floats(void) { return gs::kRecFloats; }
extern "C" int gs_grad2d_floats(void) { return gs::kGrad2D; }
