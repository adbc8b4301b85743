// Elementary functions built only from correctly rounded IEEE operations (+, -, *, fma,
// division, sqrt, rint, ldexp), so that the CPU oracle, which evaluates the same sequences,
// reproduces every result bit for bit. Hardware transcendental approximations (v_exp_f32,
// v_log_f32) are not used on the rasterizer path: their last bits are not specified.
//
//   exp2_neg / exp2_any   2^x, float; degree-6 polynomial on [-1/2, 1/2] (Chebyshev
//                         interpolant), used with a conic pre-scaled by log2(e)
//   exp_f32 / exp_f64     e^x; Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2, with the
//                         two-part ln2 of fdlibm, then the Taylor polynomial of e^r
//                         (degree 7 for float, 13 for double), then ldexp(p, k)
//   log_pos / log_f64     ln x for normal x > 0: x = 2^e m, m in [sqrt(1/2), sqrt(2)),
//                         ln m = 2 atanh(s), s = (m - 1) / (m + 1), odd series in s
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

constexpr float kLog2e = 1.44269504f;
constexpr float kNegHalfLog2e = -0.72134752f;
constexpr float kNegLog2e = -1.44269504f;
constexpr float kLn2 = 0.693147182f;
constexpr float kSqrt2 = 1.41421354f;

// ---- 2^x, float -----------------------------------------------------------------------
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

// x clamped to [lo, hi] in one instruction (x is never NaN here).
__device__ __forceinline__ float clampf(float x, float lo, float hi) { return __builtin_amdgcn_fmed3f(x, lo, hi); }

// 2^x for x clamped to [-126, 126].
__device__ __forceinline__ float exp2_any(float x) {
  x = fminf(fmaxf(x, -126.0f), 126.0f);
  const float k = rintf(x);
  const float f = x - k;
  return ldexpf(poly_exp2_frac(f), static_cast<int>(k));
}

__device__ __forceinline__ float exp_any(float x) { return exp2_any(x * kLog2e); }

__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + exp_any(-z)); }

// ---- e^x, float and double --------------------------------------------------------------
constexpr float kLn2HiF = 0.693145751953125f;       // 0x3f317200: 16 trailing zero bits
constexpr float kLn2LoF = 1.42860676533018720e-06f;  // ln2 - kLn2HiF
constexpr double kLog2eD = 1.4426950408889634;
constexpr double kLn2HiD = 6.93147180369123816490e-01;  // fdlibm ln2_hi
constexpr double kLn2LoD = 1.90821492927058770002e-10;  // fdlibm ln2_lo

__device__ __forceinline__ float exp_f32(float x) {
  if (x < -104.0f) return 0.0f;
  if (x > 88.7f) return __builtin_huge_valf();
  const float k = rintf(x * kLog2e);
  float r = fmaf(-k, kLn2HiF, x);
  r = fmaf(-k, kLn2LoF, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, static_cast<int>(k));
}

__device__ __forceinline__ double exp_f64(double x) {
  if (x < -746.0) return 0.0;
  if (x > 709.7) return __builtin_huge_val();
  const double k = rint(x * kLog2eD);
  double r = fma(-k, kLn2HiD, x);
  r = fma(-k, kLn2LoD, r);
  double p = 1.0 / 6227020800.0;  // 1/13!
  p = fma(p, r, 1.0 / 479001600.0);
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  return ldexp(p, static_cast<int>(k));
}

__device__ __forceinline__ float exp_t(float x) { return exp_f32(x); }
__device__ __forceinline__ double exp_t(double x) { return exp_f64(x); }

// ---- ln x -----------------------------------------------------------------------------
// Natural log of a positive normal float.
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

// Natural log of a positive normal double (series to s^23).
__device__ __forceinline__ double log_f64(double x) {
  const uint64_t bits = static_cast<uint64_t>(__double_as_longlong(x));
  int e = static_cast<int>((bits >> 52) & 0x7ffu) - 1023;
  double m = __longlong_as_double(static_cast<long long>((bits & 0x000fffffffffffffull) |
                                                         0x3ff0000000000000ull));
  if (m > 1.4142135623730951) {
    m = m * 0.5;
    e = e + 1;
  }
  const double s = (m - 1.0) / (m + 1.0);
  const double s2 = s * s;
  double p = 1.0 / 23.0;
  p = fma(p, s2, 1.0 / 21.0);
  p = fma(p, s2, 1.0 / 19.0);
  p = fma(p, s2, 1.0 / 17.0);
  p = fma(p, s2, 1.0 / 15.0);
  p = fma(p, s2, 1.0 / 13.0);
  p = fma(p, s2, 1.0 / 11.0);
  p = fma(p, s2, 1.0 / 9.0);
  p = fma(p, s2, 1.0 / 7.0);
  p = fma(p, s2, 1.0 / 5.0);
  p = fma(p, s2, 1.0 / 3.0);
  p = fma(p, s2, 1.0);
  double t = s * p;
  t = t + t;
  const double ed = static_cast<double>(e);
  return fma(ed, kLn2HiD, fma(ed, kLn2LoD, t));
}

template <typename S>
__device__ __forceinline__ S sigmoid_t(S z) {
  return S(1) / (S(1) + exp_t(-z));
}

}  // namespace gs
