// Rule sets of the three operator surfaces, as compile-time traits shared by the forward
// blend, the bucketed backward and the per-pixel backward (one kernel family, no second
// code path per surface):
//
//                 3D (rasterize)          toy2d (gs2d.rasterize)      phase0 (splat2d.render)
//  pixel centre   x + 0.5                 x                           x + 0.5
//  shape          conic A B C, exp2 form  conic A B C                 Cholesky l0 l1 l2 of Q
//  exponent       min(power, 0)           power, skipped if > 0       -q/2
//  alpha          o G                     min(0.99, o G)              min(0.99, o G)
//  termination    after T < 1e-4          before T (1-a) < 1e-4       after T < 1e-4
//  background     T bg                    T bg                        none
//  image          [3,H,W]                 [3,H,W]                     [H,W,3]
//  checkpoint     (C, T)                  (T, C)                      (C, T)
//  n_contrib      last position + 1       last position + 1           number of splats
//
// Sources: toy2d/csrc/rasterize.cu:37-101,146-157,171-173; toy2d/gs2d/reference.py:3-8;
// phase0/csrc/macrotile/splat2d_common.h:7-11,113-150,158-246; phase1/fastergs_macro.patch:
// 181-205; upstream/upstream_main_kernels.patch:9-13,98.
//
// Splat record in HBM (16 scalars per Gaussian, written by the preprocess or gs2d_pack):
//   0 mean.x  1 mean.y  2 A|l0  3 B|l1  4 C|l2  5 opacity  6 depth  7 ln(255 o)
//   8 r  9 g  10 b  11 clamp-mask bits (3D)  12..15 3D pixel bounds (int32 x0 x1 y0 y1)
#pragma once

#include "gs_common.h"

namespace gs {

enum RuleSet : int { kRules3D = 0, kRulesToy2D = 1, kRulesPhase0 = 2 };

// One splat as staged in LDS (all lanes read the same entry: broadcast, no conflicts).
template <typename S>
struct alignas(16) Staged {
  S mx, my;     // mean
  S s0, s1, s2;  // 3D forward: conic pre-scaled for exp2; 2D: conic or Cholesky factors
  S o;          // opacity
  S cr, cg, cb;  // colour
  S n0, n1;     // 3D: natural conic A and B (C is in nat2); 2D: unused
  S nat2;       // 3D: natural conic C
};

// Result of evaluating one splat at one pixel centre.
template <typename S>
struct Eval {
  S dx, dy;     // 3D / toy2d: mean - pixel; phase0: pixel - mean
  S G;          // Gaussian falloff
  S alpha;      // opacity after the rule's clamp
  S a, b;       // phase0: l0 dx + l1 dy and l2 dy
  bool clamped;  // alpha hit 0.99: no gradient through alpha
};

template <int R, typename S>
struct Rule;

// ---------------------------------------------------------------------------------------
template <>
struct Rule<kRules3D, float> {
  using S = float;
  static constexpr bool kStopBefore = false;
  static constexpr bool kInterleaved = false;
  static constexpr bool kCkptTFirst = false;
  static constexpr bool kCountContrib = false;
  static constexpr bool kStrips = true;
  static constexpr bool kBackground = true;
  static constexpr int kGradVals = 11;  // mean 2, conic 3, opacity, colour 3, |dmean| 2
  __device__ static S pix_off() { return 0.5f; }
  __device__ static S alpha_min() { return kAlphaMin; }
  __device__ static S t_stop() { return kTStop; }

  __device__ static Staged<S> stage(const S* r) {
    const float4 a = reinterpret_cast<const float4*>(r)[0];
    const float4 b = reinterpret_cast<const float4*>(r)[1];
    const float4 c = reinterpret_cast<const float4*>(r)[2];
    Staged<S> s;
    s.mx = a.x;
    s.my = a.y;
    s.s0 = a.z * kNegHalfLog2e;
    s.s1 = a.w * kNegLog2e;
    s.s2 = b.x * kNegHalfLog2e;
    s.o = b.y;
    s.cr = c.x;
    s.cg = c.y;
    s.cb = c.z;
    s.n0 = a.z;
    s.n1 = a.w;
    s.nat2 = b.x;
    return s;
  }

  // power (in log2 units) = s0 dx^2 + s1 dx dy + s2 dy^2, evaluated as
  // a0 + dy (s2 dy + b1) with the column terms a0 = (s0 dx) dx, b1 = s1 dx, which a lane
  // owning several pixels of one column computes once per splat; clamped to [-64, 0].
  struct Col {
    float dx, a0, b1;
  };
  __device__ static Col col(const Staged<S>& s, S px) {
    Col c;
    c.dx = s.mx - px;
    c.a0 = (s.s0 * c.dx) * c.dx;
    c.b1 = s.s1 * c.dx;
    return c;
  }
  __device__ static float power(const Staged<S>& s, const Col& c, float dy) {
    return clampf(fmaf(dy, fmaf(s.s2, dy, c.b1), c.a0), -64.0f, 0.0f);
  }
  // G = 2^power with the hardware exp2 (v_exp_f32, within 1 ulp): about a third of the
  // instructions of a polynomial exp2 in the loops that dominate the blend.
  __device__ static float falloff(float pw) { return __builtin_amdgcn_exp2f(pw); }
  __device__ static bool eval(const Staged<S>& s, S px, S py, Eval<S>& e) {
    const Col c = col(s, px);
    e.dx = c.dx;
    e.dy = s.my - py;
    e.G = falloff(power(s, c, e.dy));
    e.alpha = s.o * e.G;
    e.clamped = false;
    return e.alpha >= kAlphaMin;
  }
};

// ---------------------------------------------------------------------------------------
template <typename S>
struct Rule<kRulesToy2D, S> {
  static constexpr bool kStopBefore = true;
  static constexpr bool kInterleaved = false;
  static constexpr bool kCkptTFirst = true;
  static constexpr bool kCountContrib = false;
  static constexpr bool kStrips = false;
  static constexpr bool kBackground = true;
  static constexpr int kGradVals = 9;
  __device__ static S pix_off() { return S(0); }
  __device__ static S alpha_min() { return S(1) / S(255); }
  __device__ static S t_stop() { return S(1e-4); }

  __device__ static Staged<S> stage(const S* r) {
    Staged<S> s;
    s.mx = r[0];
    s.my = r[1];
    s.s0 = r[2];
    s.s1 = r[3];
    s.s2 = r[4];
    s.o = r[5];
    s.cr = r[8];
    s.cg = r[9];
    s.cb = r[10];
    s.n0 = s.n1 = s.nat2 = S(0);
    return s;
  }

  // power = -0.5 (A dx dx + C dy dy) - B dx dy, skipped if positive; alpha = min(0.99, o G)
  __device__ static bool eval(const Staged<S>& s, S px, S py, Eval<S>& e) {
    e.dx = s.mx - px;
    e.dy = s.my - py;
    const S t1 = (s.s0 * e.dx) * e.dx;
    const S t2 = (s.s2 * e.dy) * e.dy;
    const S power = S(-0.5) * (t1 + t2) - (s.s1 * e.dx) * e.dy;
    if (power > S(0)) return false;
    e.G = exp_t(power);
    const S raw = s.o * e.G;
    e.clamped = raw > S(0.99);
    e.alpha = e.clamped ? S(0.99) : raw;
    return e.alpha >= alpha_min();
  }
};

// ---------------------------------------------------------------------------------------
template <typename S>
struct Rule<kRulesPhase0, S> {
  static constexpr bool kStopBefore = false;
  static constexpr bool kInterleaved = true;
  static constexpr bool kCkptTFirst = false;
  static constexpr bool kCountContrib = true;
  static constexpr bool kStrips = false;
  static constexpr bool kBackground = false;
  static constexpr int kGradVals = 9;
  __device__ static S pix_off() { return S(0.5); }
  __device__ static S alpha_min() { return S(1.0 / 255.0); }
  __device__ static S t_stop() { return S(1e-4); }

  __device__ static Staged<S> stage(const S* r) { return Rule<kRulesToy2D, S>::stage(r); }

  // q = (l0 dx + l1 dy)^2 + (l2 dy)^2, G = exp(-q/2), alpha = min(0.99, o G)
  __device__ static bool eval(const Staged<S>& s, S px, S py, Eval<S>& e) {
    e.dx = px - s.mx;
    e.dy = py - s.my;
    e.a = s.s0 * e.dx + s.s1 * e.dy;
    e.b = s.s2 * e.dy;
    const S q = e.a * e.a + e.b * e.b;
    e.G = exp_t(S(-0.5) * q);
    const S raw = s.o * e.G;
    e.clamped = raw > S(0.99);
    e.alpha = e.clamped ? S(0.99) : raw;
    return e.alpha >= alpha_min();
  }
};

// Front-to-back compositing step in each rule set's operation order (the backward replays
// T with the identical update, so the replayed T is the forward's bit for bit).
template <int R, typename S>
__device__ __forceinline__ void composite(S& Cr, S& Cg, S& Cb, S& T, const Staged<S>& s, S alpha) {
  if constexpr (R == kRulesPhase0) {
    Cr = Cr + (s.cr * alpha) * T;
    Cg = Cg + (s.cg * alpha) * T;
    Cb = Cb + (s.cb * alpha) * T;
  } else {
    const S w = alpha * T;
    Cr = fma(s.cr, w, Cr);
    Cg = fma(s.cg, w, Cg);
    Cb = fma(s.cb, w, Cb);
  }
  T = T * (S(1) - alpha);
}

// Gradient of one (pixel, splat) pair with respect to the splat's screen-space parameters,
// given dL/dalpha. acc[0..1] mean, acc[2..4] shape, acc[5] opacity (dL/do; the caller
// applies o (1 - o) for logit parametrisations), acc[6..8] colour (added by the caller),
// acc[9..10] |dL/dmean| (3D only).
template <int R, typename S>
__device__ __forceinline__ void shape_grads(const Staged<S>& s, const Eval<S>& e, S dLda, S* acc) {
  if (e.clamped) return;
  acc[5] += e.G * dLda;
  const S hp = e.alpha * dLda;  // dL/dpower
  if constexpr (R == kRulesPhase0) {
    // power = -(a^2 + b^2) / 2, a = l0 dx + l1 dy, b = l2 dy, d = pixel - mean
    acc[0] += hp * e.a * s.s0;
    acc[1] += hp * (e.a * s.s1 + e.b * s.s2);
    acc[2] -= hp * e.a * e.dx;
    acc[3] -= hp * e.a * e.dy;
    acc[4] -= hp * e.b * e.dy;
  } else {
    // power = -1/2 (A dx^2 + 2 B dx dy + C dy^2), d = mean - pixel
    S A, B, C;
    if constexpr (R == kRules3D) {
      A = s.n0;
      B = s.n1;
      C = s.nat2;
    } else {
      A = s.s0;
      B = s.s1;
      C = s.s2;
    }
    acc[2] += S(-0.5) * hp * e.dx * e.dx;
    acc[3] += -hp * e.dx * e.dy;
    acc[4] += S(-0.5) * hp * e.dy * e.dy;
    const S gmx = -hp * (A * e.dx + B * e.dy);
    const S gmy = -hp * (B * e.dx + C * e.dy);
    acc[0] += gmx;
    acc[1] += gmy;
    if constexpr (R == kRules3D) {
      acc[9] += fabs(gmx);
      acc[10] += fabs(gmy);
    }
  }
}

}  // namespace gs
