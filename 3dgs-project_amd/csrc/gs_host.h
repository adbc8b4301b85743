// Host-side helpers of the C ABI: error reporting and camera set-up.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <string>

#include "../../include/amdsplat.h"
#include "gs_camera.h"

namespace gs {

void set_error(const char* fmt, ...);
void clear_error();

// Returns GS_ERR_LAUNCH (and records the message) if the last launch failed.
int check_launch(const char* what);

// Records a stage mark on `st` if stage marks are enabled on this thread (gs_stage_marks).
void stage_mark(const char* name, hipStream_t st);

// Enqueues a zero fill of n floats (a kernel, not hipMemsetAsync, so the call can be
// captured in a HIP graph).
void fill_zero_f32(float* p, int64_t n, hipStream_t st);

#define GS_REQUIRE(cond, code, ...) \
  do {                              \
    if (!(cond)) {                  \
      ::gs::set_error(__VA_ARGS__); \
      return (code);                \
    }                               \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Host twin of float_order_key (the 32-bit key whose unsigned order is the float order).
inline uint32_t host_order_key(float v) {
  uint32_t u;
  v = v + 0.0f;
  memcpy(&u, &v, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Bits the 3D depth sort needs for the keys of gs_preprocess_fwd (see CamK::dkey_cull).
inline int depth_key_bits(const CamK& k) {
  int b = 0;
  while (b < 32 && (k.dkey_cull >> b) != 0u) ++b;
  return b;
}

// Builds the kernel camera. Derived values are computed in double and rounded once, the
// same way the CPU oracle derives them.
inline CamK make_cam(const gs_camera& c) {
  CamK k;
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 3; ++j) k.r[3 * i + j] = c.viewmat[4 * i + j];
    k.t[i] = c.viewmat[4 * i + 3];
  }
  k.fx = c.fx;
  k.fy = c.fy;
  k.cx = c.cx;
  k.cy = c.cy;
  k.width = c.width;
  k.height = c.height;
  k.znear = c.near_plane;
  k.zfar = c.far_plane;
  k.flags = c.flags;
  for (int j = 0; j < 3; ++j) {
    double s = 0.0;
    for (int i = 0; i < 3; ++i) s -= static_cast<double>(c.viewmat[4 * i + j]) * c.viewmat[4 * i + 3];
    k.campos[j] = static_cast<float>(s);
  }
  k.lim_x_lo = static_cast<float>(-1.3 * static_cast<double>(c.cx) / c.fx);
  k.lim_x_hi = static_cast<float>(1.3 * (static_cast<double>(c.width) - c.cx) / c.fx);
  k.lim_y_lo = static_cast<float>(-1.3 * static_cast<double>(c.cy) / c.fy);
  k.lim_y_hi = static_cast<float>(1.3 * (static_cast<double>(c.height) - c.cy) / c.fy);
  k.tiles_x = (c.width + kTile - 1) / kTile;
  k.tiles_y = (c.height + kTile - 1) / kTile;
  k.dkey0 = host_order_key(c.near_plane);
  k.dkey_cull = host_order_key(c.far_plane) - k.dkey0;
  return k;
}

inline int check_cam(const gs_camera* c) {
  GS_REQUIRE(c != nullptr, GS_ERR_ARG, "camera is NULL");
  GS_REQUIRE(c->width > 0 && c->height > 0 && c->width <= 32768 && c->height <= 32768, GS_ERR_ARG,
             "image size %dx%d out of range", c->width, c->height);
  GS_REQUIRE(c->near_plane > 0.0f && c->far_plane > c->near_plane, GS_ERR_ARG,
             "need 0 < near < far (got %g, %g)", c->near_plane, c->far_plane);
  GS_REQUIRE(c->fx > 0.0f && c->fy > 0.0f, GS_ERR_ARG, "focal lengths must be positive");
  return GS_OK;
}

}  // namespace gs
