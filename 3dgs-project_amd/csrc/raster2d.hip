// 2D surfaces: tile rectangles of the two 2D binning rules and the splat-record pack.
//
//  toy2d   rect = getRect of the 3-sigma radius, in float32 like the caller's torch ops
//          (toy2d/gs2d/binning.py:44-57): min = trunc((m - r) / 16), max = trunc((m + r + 15) / 16)
//          evaluated as ((m + r) + 16) - 1, both clamped to the grid; radius <= 0 or an empty
//          rectangle touches nothing.
//  phase0  rect = tiles of the alpha >= 1/255 ellipse's bounding box plus one pixel of slack,
//          in float64 (phase0/splat2d/ops.py:209-235): r^2 = 2 ln(255 o),
//          ex = r sqrt(1/l0^2 + (l1/(l0 l2))^2), ey = r/|l2|, x0 = floor(m - ex - 0.5) - 1,
//          x1 = ceil(m + ex - 0.5) + 1 (same for y); kept if r^2 > 0 and the box meets the image.
#include "gs_host.h"
#include "gs_rules.h"

namespace gs {

__global__ void rects_toy_kernel(const float2* __restrict__ means, const int32_t* __restrict__ radii, int64_t n,
                                 int tiles_x, int tiles_y, int4* __restrict__ rects,
                                 uint32_t* __restrict__ counts) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float2 m = means[i];
  const int32_t rad = radii[i];
  const float r = static_cast<float>(rad);
  const float tf = static_cast<float>(kTile);
  const float fx = static_cast<float>(tiles_x), fy = static_cast<float>(tiles_y);
  const int xmin = static_cast<int>(fminf(fmaxf(truncf((m.x - r) / tf), 0.0f), fx));
  const int ymin = static_cast<int>(fminf(fmaxf(truncf((m.y - r) / tf), 0.0f), fy));
  const int xmax = static_cast<int>(fminf(fmaxf(truncf((((m.x + r) + tf) - 1.0f) / tf), 0.0f), fx));
  const int ymax = static_cast<int>(fminf(fmaxf(truncf((((m.y + r) + tf) - 1.0f) / tf), 0.0f), fy));
  const int w = rad > 0 ? xmax - xmin : 0;
  const int h = rad > 0 ? ymax - ymin : 0;
  const int64_t c = static_cast<int64_t>(w) * h;
  const bool empty = c <= 0;
  rects[i] = make_int4(xmin, ymin, empty ? xmin : xmax, empty ? ymin : ymax);
  counts[i] = empty ? 0u : static_cast<uint32_t>(c);
}

template <typename S>
__global__ void rects_phase0_kernel(const S* __restrict__ means, const S* __restrict__ chol,
                                    const S* __restrict__ logit, int64_t n, int W, int H, int4* __restrict__ rects,
                                    uint32_t* __restrict__ counts) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double mx = static_cast<double>(means[2 * i]), my = static_cast<double>(means[2 * i + 1]);
  const double l0 = static_cast<double>(chol[3 * i]), l1 = static_cast<double>(chol[3 * i + 1]);
  const double l2 = static_cast<double>(chol[3 * i + 2]);
  const double o = sigmoid_t(static_cast<double>(logit[i]));
  const double r2 = 2.0 * log_f64(255.0 * o);
  const double r = sqrt(fmax(r2, 0.0));
  const double q = l1 / (l0 * l2);
  const double ex = r * sqrt(1.0 / (l0 * l0) + q * q);
  const double ey = r / fabs(l2);
  const double x0 = floor((mx - ex) - 0.5) - 1.0;
  const double x1 = ceil((mx + ex) - 0.5) + 1.0;
  const double y0 = floor((my - ey) - 0.5) - 1.0;
  const double y1 = ceil((my + ey) - 0.5) + 1.0;
  const double wm = static_cast<double>(W - 1), hm = static_cast<double>(H - 1);
  const bool valid = (r2 > 0.0) && (x1 >= 0.0) && (x0 <= wm) && (y1 >= 0.0) && (y0 <= hm);
  if (!valid) {
    rects[i] = make_int4(0, 0, 0, 0);
    counts[i] = 0u;
    return;
  }
  const int tx0 = static_cast<int>(floor(fmin(fmax(x0, 0.0), wm) / kTile));
  const int tx1 = static_cast<int>(floor(fmin(fmax(x1, 0.0), wm) / kTile));
  const int ty0 = static_cast<int>(floor(fmin(fmax(y0, 0.0), hm) / kTile));
  const int ty1 = static_cast<int>(floor(fmin(fmax(y1, 0.0), hm) / kTile));
  rects[i] = make_int4(tx0, ty0, tx1 + 1, ty1 + 1);
  counts[i] = static_cast<uint32_t>((tx1 - tx0 + 1) * (ty1 - ty0 + 1));
}

// Record of one 2D Gaussian (layout in gs_rules.h).
template <int R, typename S>
__global__ void pack_kernel(const S* __restrict__ means, const S* __restrict__ shape, const S* __restrict__ color,
                            const S* __restrict__ opacity, int64_t n, S* __restrict__ rec) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  S v[kRecFloats];
  v[0] = means[2 * i];
  v[1] = means[2 * i + 1];
  v[2] = shape[3 * i];
  v[3] = shape[3 * i + 1];
  v[4] = shape[3 * i + 2];
  if constexpr (R == kRulesPhase0) {
    v[5] = sigmoid_t(opacity[i]);  // opacity logit -> opacity (splat2d_common.h:116)
    v[6] = opacity[i];
  } else {
    v[5] = opacity[i];
    v[6] = S(0);
  }
  v[7] = S(0);
  v[8] = color[3 * i];
  v[9] = color[3 * i + 1];
  v[10] = color[3 * i + 2];
  for (int k = 11; k < kRecFloats; ++k) v[k] = S(0);
  S* dst = rec + i * kRecFloats;
  for (int k = 0; k < kRecFloats; ++k) dst[k] = v[k];
}

// The toy2d activation (toy2d/gs2d/params.py:36-46) of Gaussian i, in the reference's operation
// order (each product and sum rounded on its own, as separate tensor operations round them):
// var = exp(2 log_scale), cxx = c c vx + s s vy, cxy = c s (vx - vy), cyy = s s vx + c c vy with
// (c, s) = (cos, sin)(theta), det = cxx cyy - cxy cxy, conic = (cyy, -cxy, cxx) / det; and the
// integer 3-sigma radius of toy2d/gs2d/params.py:49-56 (0 where det <= 0).
struct Act2D {
  float vx, vy, c, s, cxx, cxy, cyy, det;
};

__device__ __forceinline__ Act2D activate2d(const float* __restrict__ log_scale, const float* __restrict__ theta,
                                            int64_t i) {
  Act2D a;
  a.vx = expf(2.0f * log_scale[2 * i]);
  a.vy = expf(2.0f * log_scale[2 * i + 1]);
  a.c = cosf(theta[i]);
  a.s = sinf(theta[i]);
  const float cc = a.c * a.c, ss = a.s * a.s;
  a.cxx = cc * a.vx + ss * a.vy;
  a.cxy = (a.c * a.s) * (a.vx - a.vy);
  a.cyy = ss * a.vx + cc * a.vy;
  a.det = a.cxx * a.cyy - a.cxy * a.cxy;
  return a;
}

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ void activate2d_fwd_kernel(const float* __restrict__ log_scale, const float* __restrict__ theta,
                                      const float* __restrict__ rgb_logit, const float* __restrict__ opacity_logit,
                                      int64_t n, float* __restrict__ conic, float* __restrict__ color,
                                      float* __restrict__ opacity, float* __restrict__ cov,
                                      int32_t* __restrict__ radii) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const Act2D a = activate2d(log_scale, theta, i);
  conic[3 * i] = a.cyy / a.det;
  conic[3 * i + 1] = -a.cxy / a.det;
  conic[3 * i + 2] = a.cxx / a.det;
  for (int k = 0; k < 3; ++k) color[3 * i + k] = sigmoid_ref(rgb_logit[3 * i + k]);
  opacity[i] = sigmoid_ref(opacity_logit[i]);
  if (cov) {
    cov[3 * i] = a.cxx;
    cov[3 * i + 1] = a.cxy;
    cov[3 * i + 2] = a.cyy;
  }
  if (radii) {
    const float mid = 0.5f * (a.cxx + a.cyy);
    const float lam = mid + sqrtf(fmaxf(mid * mid - a.det, 0.1f));
    radii[i] = a.det > 0.0f ? static_cast<int32_t>(ceilf(3.0f * sqrtf(lam))) : 0;
  }
}

// Gradients of the activation from those of conic, colour and opacity (means pass through): the
// chain rule through conic = (cyy, -cxy, cxx) / det, the covariance and exp / cos / sin, with the
// forward's values recomputed; colour and opacity through the sigmoid, s (1 - s).
__global__ void activate2d_bwd_kernel(const float* __restrict__ log_scale, const float* __restrict__ theta,
                                      const float* __restrict__ rgb_logit, const float* __restrict__ opacity_logit,
                                      int64_t n, const float* __restrict__ g_conic, const float* __restrict__ g_color,
                                      const float* __restrict__ g_opacity, float* __restrict__ g_log_scale,
                                      float* __restrict__ g_theta, float* __restrict__ g_rgb_logit,
                                      float* __restrict__ g_opacity_logit) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const Act2D a = activate2d(log_scale, theta, i);
  const float gA = g_conic ? g_conic[3 * i] : 0.0f, gB = g_conic ? g_conic[3 * i + 1] : 0.0f;
  const float gC = g_conic ? g_conic[3 * i + 2] : 0.0f;
  const float id = 1.0f / a.det;
  // K = (gA cyy - gB cxy + gC cxx) / det^2 = d L / d(1 / det) / ... : the det term of every entry
  const float K = (gA * a.cyy - gB * a.cxy + gC * a.cxx) * id * id;
  const float g_cxx = gC * id - K * a.cyy;
  const float g_cyy = gA * id - K * a.cxx;
  const float g_cxy = -gB * id + 2.0f * K * a.cxy;
  const float cc = a.c * a.c, ss = a.s * a.s, cs = a.c * a.s, dv = a.vx - a.vy;
  const float g_vx = g_cxx * cc + g_cxy * cs + g_cyy * ss;
  const float g_vy = g_cxx * ss - g_cxy * cs + g_cyy * cc;
  const float g_c = 2.0f * a.c * (g_cxx * a.vx + g_cyy * a.vy) + g_cxy * a.s * dv;
  const float g_s = 2.0f * a.s * (g_cxx * a.vy + g_cyy * a.vx) + g_cxy * a.c * dv;
  g_log_scale[2 * i] = 2.0f * a.vx * g_vx;
  g_log_scale[2 * i + 1] = 2.0f * a.vy * g_vy;
  g_theta[i] = a.c * g_s - a.s * g_c;
  for (int k = 0; k < 3; ++k) {
    const float sg = sigmoid_ref(rgb_logit[3 * i + k]);
    g_rgb_logit[3 * i + k] = g_color ? g_color[3 * i + k] * sg * (1.0f - sg) : 0.0f;
  }
  const float so = sigmoid_ref(opacity_logit[i]);
  g_opacity_logit[i] = g_opacity ? g_opacity[i] * so * (1.0f - so) : 0.0f;
}

}  // namespace gs

using namespace gs;

static inline unsigned grid256(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

extern "C" int gs2d_activate_fwd(const float* log_scale, const float* theta, const float* rgb_logit,
                                 const float* opacity_logit, int64_t n, float* conic, float* color, float* opacity,
                                 float* cov, int32_t* radii, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_ARG, "n must be >= 0");
  if (n == 0) return GS_OK;
  GS_REQUIRE(log_scale && theta && rgb_logit && opacity_logit && conic && color && opacity, GS_ERR_ARG,
             "null pointer argument");
  hipLaunchKernelGGL(activate2d_fwd_kernel, dim3(grid256(n)), dim3(256), 0, as_stream(stream), log_scale, theta,
                     rgb_logit, opacity_logit, n, conic, color, opacity, cov, radii);
  return check_launch("gs2d_activate_fwd");
}

extern "C" int gs2d_activate_bwd(const float* log_scale, const float* theta, const float* rgb_logit,
                                 const float* opacity_logit, int64_t n, const float* grad_conic,
                                 const float* grad_color, const float* grad_opacity, float* grad_log_scale,
                                 float* grad_theta, float* grad_rgb_logit, float* grad_opacity_logit,
                                 void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_ARG, "n must be >= 0");
  if (n == 0) return GS_OK;
  GS_REQUIRE(log_scale && theta && rgb_logit && opacity_logit && grad_log_scale && grad_theta && grad_rgb_logit &&
                 grad_opacity_logit,
             GS_ERR_ARG, "null pointer argument");
  hipLaunchKernelGGL(activate2d_bwd_kernel, dim3(grid256(n)), dim3(256), 0, as_stream(stream), log_scale, theta,
                     rgb_logit, opacity_logit, n, grad_conic, grad_color, grad_opacity, grad_log_scale, grad_theta,
                     grad_rgb_logit, grad_opacity_logit);
  return check_launch("gs2d_activate_bwd");
}

extern "C" int gs2d_rects_toy(const float* means, const int32_t* radii, int64_t n, int width, int height,
                              int32_t* rects, uint32_t* counts, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && width > 0 && height > 0, GS_ERR_ARG, "invalid sizes");
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && radii && rects && counts, GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(means, 8) && aligned(rects, 16), GS_ERR_ALIGN,
             "means must be 8-byte and rects 16-byte aligned");
  const int tiles_x = (width + kTile - 1) / kTile, tiles_y = (height + kTile - 1) / kTile;
  hipLaunchKernelGGL(rects_toy_kernel, dim3(grid256(n)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const float2*>(means), radii, n, tiles_x, tiles_y,
                     reinterpret_cast<int4*>(rects), counts);
  return check_launch("gs2d_rects_toy");
}

extern "C" int gs2d_rects_phase0(int dtype, const void* means, const void* chol, const void* opacity_logit,
                                 int64_t n, int width, int height, int32_t* rects, uint32_t* counts,
                                 void* stream) {
  clear_error();
  GS_REQUIRE(dtype == GS_FLOAT32 || dtype == GS_FLOAT64, GS_ERR_ARG, "invalid dtype %d", dtype);
  GS_REQUIRE(n >= 0 && width > 0 && height > 0, GS_ERR_ARG, "invalid sizes");
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && chol && opacity_logit && rects && counts, GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(rects, 16), GS_ERR_ALIGN, "rects must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  if (dtype == GS_FLOAT32) {
    hipLaunchKernelGGL(rects_phase0_kernel<float>, dim3(grid256(n)), dim3(256), 0, st,
                       static_cast<const float*>(means), static_cast<const float*>(chol),
                       static_cast<const float*>(opacity_logit), n, width, height, reinterpret_cast<int4*>(rects),
                       counts);
  } else {
    hipLaunchKernelGGL(rects_phase0_kernel<double>, dim3(grid256(n)), dim3(256), 0, st,
                       static_cast<const double*>(means), static_cast<const double*>(chol),
                       static_cast<const double*>(opacity_logit), n, width, height,
                       reinterpret_cast<int4*>(rects), counts);
  }
  return check_launch("gs2d_rects_phase0");
}

// Gradient record [n, 12] -> dmeans [n, 2], dshape [n, 3], dopacity [n], dcolor [n, 3] (slots 0-1,
// 2-4, 5, 6-8), a thread per splat.
template <typename S>
__global__ void unpack_grads_kernel(const S* __restrict__ g, int64_t n, S* __restrict__ dm, S* __restrict__ ds,
                                    S* __restrict__ dop, S* __restrict__ dc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const S* r = g + i * kGrad2D;
  dm[2 * i] = r[0];
  dm[2 * i + 1] = r[1];
  ds[3 * i] = r[2];
  ds[3 * i + 1] = r[3];
  ds[3 * i + 2] = r[4];
  dop[i] = r[5];
  dc[3 * i] = r[6];
  dc[3 * i + 1] = r[7];
  dc[3 * i + 2] = r[8];
}

extern "C" int gs2d_unpack_grads(int dtype, const void* grad_rec, int64_t n, void* dmeans, void* dshape,
                                 void* dopacity, void* dcolor, void* stream) {
  clear_error();
  GS_REQUIRE(dtype == GS_FLOAT32 || dtype == GS_FLOAT64, GS_ERR_ARG, "invalid dtype %d", dtype);
  GS_REQUIRE(n >= 0, GS_ERR_ARG, "invalid size");
  if (n == 0) return GS_OK;
  GS_REQUIRE(grad_rec && dmeans && dshape && dopacity && dcolor, GS_ERR_ARG, "null pointer argument");
  hipStream_t st = as_stream(stream);
  if (dtype == GS_FLOAT32)
    hipLaunchKernelGGL(unpack_grads_kernel<float>, dim3(grid256(n)), dim3(256), 0, st,
                       static_cast<const float*>(grad_rec), n, static_cast<float*>(dmeans),
                       static_cast<float*>(dshape), static_cast<float*>(dopacity), static_cast<float*>(dcolor));
  else
    hipLaunchKernelGGL(unpack_grads_kernel<double>, dim3(grid256(n)), dim3(256), 0, st,
                       static_cast<const double*>(grad_rec), n, static_cast<double*>(dmeans),
                       static_cast<double*>(dshape), static_cast<double*>(dopacity), static_cast<double*>(dcolor));
  return check_launch("gs2d_unpack_grads");
}

extern "C" int gs2d_pack(int rules, int dtype, const void* means, const void* shape, const void* color,
                         const void* opacity, int64_t n, void* rec, void* stream) {
  clear_error();
  GS_REQUIRE(rules == GS_RULES_TOY2D || rules == GS_RULES_PHASE0, GS_ERR_ARG, "invalid rules %d", rules);
  GS_REQUIRE(dtype == GS_FLOAT32 || dtype == GS_FLOAT64, GS_ERR_ARG, "invalid dtype %d", dtype);
  GS_REQUIRE(n >= 0, GS_ERR_ARG, "invalid size");
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && shape && color && opacity && rec, GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(rec, 16), GS_ERR_ALIGN, "rec must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
#define GS_PACK(R, S)                                                                                    \
  hipLaunchKernelGGL((pack_kernel<R, S>), dim3(grid256(n)), dim3(256), 0, st, static_cast<const S*>(means), \
                     static_cast<const S*>(shape), static_cast<const S*>(color),                          \
                     static_cast<const S*>(opacity), n, static_cast<S*>(rec))
  if (rules == GS_RULES_TOY2D) {
    if (dtype == GS_FLOAT32) GS_PACK(kRulesToy2D, float);
    else GS_PACK(kRulesToy2D, double);
  } else {
    if (dtype == GS_FLOAT32) GS_PACK(kRulesPhase0, float);
    else GS_PACK(kRulesPhase0, double);
  }
#undef GS_PACK
  return check_launch("gs2d_pack");
}
