// Real spherical-harmonics basis up to degree 3 (the 3DGS colour model) and its gradient.
// Constants are the orthonormal real-SH normalisations sqrt((2l+1)/(4 pi) (l-|m|)!/(l+|m|)!)
// times the usual Cartesian factors, with the 3DGS sign convention (band-1 terms
// -C1 y, C1 z, -C1 x; see upstream/upstream_main_kernels.patch and phase2/sh_coalesce.patch,
// convert_sh_to_color_backward_row, for the same basis in tiny-cuda-nn form).
#pragma once

#include "gs_common.h"

namespace gs {

constexpr float kSH0 = 0.28209479177387814f;
constexpr float kSH1 = 0.4886025119029199f;
constexpr float kSH2_0 = 1.0925484305920792f;
constexpr float kSH2_1 = -1.0925484305920792f;
constexpr float kSH2_2 = 0.31539156525252005f;
constexpr float kSH2_3 = -1.0925484305920792f;
constexpr float kSH2_4 = 0.5462742152960396f;
constexpr float kSH3_0 = -0.5900435899266435f;
constexpr float kSH3_1 = 2.890611442640554f;
constexpr float kSH3_2 = -0.4570457994644658f;
constexpr float kSH3_3 = 0.3731763325901154f;
constexpr float kSH3_4 = -0.4570457994644658f;
constexpr float kSH3_5 = 1.445305721320277f;
constexpr float kSH3_6 = -0.5900435899266435f;

// Basis values b[0..n) for a unit direction (x, y, z); n in {1, 4, 9, 16}.
__device__ __forceinline__ void sh_basis(float x, float y, float z, int n, float* b) {
  b[0] = kSH0;
  if (n <= 1) return;
  b[1] = -kSH1 * y;
  b[2] = kSH1 * z;
  b[3] = -kSH1 * x;
  if (n <= 4) return;
  const float xx = x * x, yy = y * y, zz = z * z;
  const float xy = x * y, yz = y * z, xz = x * z;
  b[4] = kSH2_0 * xy;
  b[5] = kSH2_1 * yz;
  {
    float t = zz + zz;
    t = t - xx;
    t = t - yy;
    b[6] = kSH2_2 * t;
  }
  b[7] = kSH2_3 * xz;
  b[8] = kSH2_4 * (xx - yy);
  if (n <= 9) return;
  b[9] = (kSH3_0 * y) * fmaf(3.0f, xx, -yy);
  b[10] = (kSH3_1 * xy) * z;
  b[11] = (kSH3_2 * y) * (fmaf(4.0f, zz, -xx) - yy);
  {
    float t = zz + zz;
    t = fmaf(-3.0f, xx, t);
    t = fmaf(-3.0f, yy, t);
    b[12] = (kSH3_3 * z) * t;
  }
  b[13] = (kSH3_4 * x) * (fmaf(4.0f, zz, -xx) - yy);
  b[14] = (kSH3_5 * z) * (xx - yy);
  b[15] = (kSH3_6 * x) * fmaf(-3.0f, yy, xx);
}

// Accumulates sum_k g[k] * grad(b_k) into (gx, gy, gz); g[k] = dL/db_k.
__device__ __forceinline__ void sh_basis_grad(float x, float y, float z, int n, const float* g,
                                              float& gx, float& gy, float& gz) {
  gx = 0.0f;
  gy = 0.0f;
  gz = 0.0f;
  if (n <= 1) return;
  gy += -kSH1 * g[1];
  gz += kSH1 * g[2];
  gx += -kSH1 * g[3];
  if (n <= 4) return;
  const float xx = x * x, yy = y * y, zz = z * z;
  const float xy = x * y, yz = y * z, xz = x * z;
  gx += kSH2_0 * y * g[4];
  gy += kSH2_0 * x * g[4];
  gy += kSH2_1 * z * g[5];
  gz += kSH2_1 * y * g[5];
  gx += -2.0f * kSH2_2 * x * g[6];
  gy += -2.0f * kSH2_2 * y * g[6];
  gz += 4.0f * kSH2_2 * z * g[6];
  gx += kSH2_3 * z * g[7];
  gz += kSH2_3 * x * g[7];
  gx += 2.0f * kSH2_4 * x * g[8];
  gy += -2.0f * kSH2_4 * y * g[8];
  if (n <= 9) return;
  gx += kSH3_0 * 6.0f * xy * g[9];
  gy += kSH3_0 * 3.0f * (xx - yy) * g[9];
  gx += kSH3_1 * yz * g[10];
  gy += kSH3_1 * xz * g[10];
  gz += kSH3_1 * xy * g[10];
  gx += kSH3_2 * -2.0f * xy * g[11];
  gy += kSH3_2 * (4.0f * zz - xx - 3.0f * yy) * g[11];
  gz += kSH3_2 * 8.0f * yz * g[11];
  gx += kSH3_3 * -6.0f * xz * g[12];
  gy += kSH3_3 * -6.0f * yz * g[12];
  gz += kSH3_3 * (6.0f * zz - 3.0f * xx - 3.0f * yy) * g[12];
  gx += kSH3_4 * (4.0f * zz - 3.0f * xx - yy) * g[13];
  gy += kSH3_4 * -2.0f * xy * g[13];
  gz += kSH3_4 * 8.0f * xz * g[13];
  gx += kSH3_5 * 2.0f * xz * g[14];
  gy += kSH3_5 * -2.0f * yz * g[14];
  gz += kSH3_5 * (xx - yy) * g[14];
  gx += kSH3_6 * 3.0f * (xx - yy) * g[15];
  gy += kSH3_6 * -6.0f * xy * g[15];
}

}  // namespace gs
