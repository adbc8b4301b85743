// Camera description shared by the 3D kernels and the exact ellipse / tile-rectangle test
// used both to count a Gaussian's tiles in the preprocess and to emit its instances in the
// binning. Both callers go through ellipse_hits_rect(), so the count and the emitted keys
// always agree.
#pragma once

#include "gs_common.h"

namespace gs {

// Kernel-side camera, passed by value. Derived quantities (camera centre, Jacobian clamp
// limits) are computed once on the host in double precision.
struct CamK {
  float r[9];    // world-to-camera rotation, row-major
  float t[3];    // world-to-camera translation
  float fx, fy, cx, cy;
  int width, height;
  float znear, zfar;
  float campos[3];       // camera centre in world space
  float lim_x_lo, lim_x_hi, lim_y_lo, lim_y_hi;  // clamp of x/z and y/z for the EWA Jacobian
  int tiles_x, tiles_y;
};

// 1/2 (A dx^2 + 2 B dx dy + C dy^2) with a fixed operation order.
__device__ __forceinline__ float half_quad(float A, float B, float C, float dx, float dy) {
  float u = C * dy;
  u = u * dy;
  float v = B * dx;
  v = v + v;
  u = fmaf(v, dy, u);
  const float w = A * dx;
  u = fmaf(w, dx, u);
  return 0.5f * u;
}

// Does the ellipse 1/2 d^T Q d <= thr (d = mean - p) reach any point p of the axis-aligned
// rectangle [X0, X1] x [Y0, Y1]? Exact for a convex quadratic: if the mean lies outside, the
// minimum over the rectangle is attained on an edge facing the mean, and on an edge the
// 1D minimiser is the clamped stationary point.
__device__ __forceinline__ bool ellipse_hits_rect(float mx, float my, float A, float B, float C,
                                                  float thr, float X0, float X1, float Y0,
                                                  float Y1) {
  const bool out_x = (mx < X0) || (mx > X1);
  const bool out_y = (my < Y0) || (my > Y1);
  if (!out_x && !out_y) return true;
  float best = 3.0e38f;
  if (out_x) {
    const float xe = (mx < X0) ? X0 : X1;
    const float dx = mx - xe;
    const float k = B / C;
    const float ys = fminf(fmaxf(fmaf(k, dx, my), Y0), Y1);
    const float dy = my - ys;
    best = fminf(best, half_quad(A, B, C, dx, dy));
  }
  if (out_y) {
    const float ye = (my < Y0) ? Y0 : Y1;
    const float dy = my - ye;
    const float k = B / A;
    const float xs = fminf(fmaxf(fmaf(k, dy, mx), X0), X1);
    const float dx = mx - xs;
    best = fminf(best, half_quad(A, B, C, dx, dy));
  }
  return best <= thr;
}

// Visits every tile whose pixels (restricted to the splat's pixel bounds) the ellipse
// reaches, in row-major tile order. Returns the number of such tiles.
template <typename F>
__device__ __forceinline__ int for_each_touched_tile(const float4 a, const float4 b, const int4 d,
                                                     int tiles_x, F&& visit) {
  const float mx = a.x, my = a.y, A = a.z, B = a.w, C = b.x, thr = b.w;
  const int tx0 = d.x / kTile, tx1 = d.y / kTile;
  const int ty0 = d.z / kTile, ty1 = d.w / kTile;
  int count = 0;
  for (int ty = ty0; ty <= ty1; ++ty) {
    const int py0 = max(ty * kTile, d.z), py1 = min(ty * kTile + kTile - 1, d.w);
    const float Y0 = static_cast<float>(py0) + 0.5f, Y1 = static_cast<float>(py1) + 0.5f;
    for (int tx = tx0; tx <= tx1; ++tx) {
      const int px0 = max(tx * kTile, d.x), px1 = min(tx * kTile + kTile - 1, d.y);
      const float X0 = static_cast<float>(px0) + 0.5f, X1 = static_cast<float>(px1) + 0.5f;
      if (ellipse_hits_rect(mx, my, A, B, C, thr, X0, X1, Y0, Y1)) {
        visit(ty * tiles_x + tx, count);
        ++count;
      }
    }
  }
  return count;
}

}  // namespace gs
