// Shared device-side definitions for the gfx950 Gaussian-splat kernels.
//
// Numerics policy. Every decision the rasterizer takes (tile membership, alpha >= 1/255,
// early termination) must come out the same on the GPU and in the CPU oracle, so the
// forward path uses only correctly rounded IEEE operations: +, -, *, fmaf, IEEE division
// and sqrt, rint and ldexp. Transcendentals are evaluated by the polynomial routines
// below instead of the hardware v_exp_f32 / v_log_f32 approximations, whose last bits are
// not specified. The library is compiled with -ffp-contract=off, so every fused
// multiply-add is an explicit fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

// ---------------------------------------------------------------------------------------
// Geometry of the tiling.
// ---------------------------------------------------------------------------------------
constexpr int kTile = 16;                    // tile side in pixels
constexpr int kTilePixels = kTile * kTile;   // 256 pixels = one forward workgroup
constexpr int kBucket = 32;                  // list entries per bucket (checkpoint stride)
constexpr int kWave = 64;                    // CDNA wavefront
constexpr int kStripRows = kWave / kTile;    // 4 tile rows per wavefront
constexpr int kStrips = kTile / kStripRows;  // 4 strips per tile
constexpr int kPixPerLane = kTilePixels / kWave;  // 4 pixels per lane in the bucket backward

constexpr float kAlphaMin = 1.0f / 255.0f;
constexpr float kTStop = 1e-4f;
constexpr float kAlphaMax2D = 0.99f;          // 2D rule sets clamp alpha at 0.99
constexpr float kOneMinusAlphaEps = 1e-6f;    // 3D backward floors (1 - alpha)
constexpr float kDilation = 0.3f;             // screen-space low-pass added to cov2d

constexpr float kLog2e = 1.44269504f;
constexpr float kNegHalfLog2e = -0.72134752f;
constexpr float kNegLog2e = -1.44269504f;
constexpr float kLn2 = 0.693147182f;
constexpr float kSqrt2 = 1.41421354f;

// Degree-6 polynomial for 2^f on [-0.5, 0.5] (Chebyshev interpolant, float32 Horner error
// below 0.7 ulp).
constexpr float kP0 = 1.0f;
constexpr float kP1 = 0.6931471824645996f;
constexpr float kP2 = 0.24022650718688965f;
constexpr float kP3 = 0.05550327152013779f;
constexpr float kP4 = 0.00961802527308464f;
constexpr float kP5 = 0.0013400432653725147f;
constexpr float kP6 = 0.00015469732170458883f;

__device__ __forceinline__ float poly_exp2_frac(float f) {
  float p = kP6;
  p = fmaf(p, f, kP5);
  p = fmaf(p, f, kP4);
  p = fmaf(p, f, kP3);
  p = fmaf(p, f, kP2);
  p = fmaf(p, f, kP1);
  p = fmaf(p, f, kP0);
  return p;
}

// 2^x for x <= 0, with x clamped at -64 so the result stays a normal float.
__device__ __forceinline__ float exp2_neg(float x) {
  x = fmaxf(x, -64.0f);
  const float k = rintf(x);
  const float f = x - k;  // exact: |f| <= 0.5
  return ldexpf(poly_exp2_frac(f), static_cast<int>(k));
}

// 2^x for x clamped to [-126, 126].
__device__ __forceinline__ float exp2_any(float x) {
  x = fminf(fmaxf(x, -126.0f), 126.0f);
  const float k = rintf(x);
  const float f = x - k;
  return ldexpf(poly_exp2_frac(f), static_cast<int>(k));
}

__device__ __forceinline__ float exp_any(float x) { return exp2_any(x * kLog2e); }

__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + exp_any(-z)); }

// Natural log of a positive normal float: x = 2^e m, m in [sqrt(1/2), sqrt(2)],
// ln m = 2 atanh(s) with s = (m - 1) / (m + 1), |s| <= 0.1716, series to s^9.
__device__ __forceinline__ float log_pos(float x) {
  const uint32_t bits = __float_as_uint(x);
  int e = static_cast<int>((bits >> 23) & 0xffu) - 127;
  float m = __uint_as_float((bits & 0x007fffffu) | 0x3f800000u);
  if (m > kSqrt2) {
    m = m * 0.5f;
    e = e + 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 1.0f / 9.0f;
  p = fmaf(p, s2, 1.0f / 7.0f);
  p = fmaf(p, s2, 1.0f / 5.0f);
  p = fmaf(p, s2, 1.0f / 3.0f);
  p = fmaf(p, s2, 1.0f);
  float t = s * p;
  t = t + t;
  return fmaf(static_cast<float>(e), kLn2, t);
}

// ---------------------------------------------------------------------------------------
// 3D splat record written by the preprocess (64 bytes, one per Gaussian):
//   a = (mean2d.x, mean2d.y, conic.A, conic.B)   power = -1/2 (A dx^2 + 2 B dx dy + C dy^2)
//   b = (conic.C, opacity, view depth, power threshold ln(255 o))
//   c = (r, g, b, clamp mask bits)   colour after SH, clamped at 0; bit k set = channel k clamped
//   d = (x0, x1, y0, y1)             inclusive pixel bounds of the alpha >= 1/255 ellipse
// ---------------------------------------------------------------------------------------
struct alignas(16) SplatRec {
  float4 a;
  float4 b;
  float4 c;
  int4 d;
};
static_assert(sizeof(SplatRec) == 64, "splat record is 64 bytes");
constexpr int kRecFloats = 16;

// Per-Gaussian screen-space gradient record accumulated by the blend backward (48 bytes):
//   [0,1] dL/dmean2d, [2,3,4] dL/d(A,B,C), [5] dL/dopacity, [6,7,8] dL/dcolour,
//   [9,10] sum over pixels of |dL/dmean2d| (densification statistic), [11] unused
constexpr int kGrad2D = 12;

// Orderable 32-bit image of a float: unsigned order equals float order.
__device__ __forceinline__ uint32_t float_order_key(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int div_up(int a, int b) { return (a + b - 1) / b; }

__device__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Makes this wavefront's earlier LDS writes visible to its other lanes (no workgroup barrier:
// wavefronts of a workgroup may have exited).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace gs
