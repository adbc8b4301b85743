// Fused L1 + D-SSIM training loss, forward and backward, on [C, H, W] float32 images:
//   L = (1 - lambda) mean|x - y| + lambda (1 - mean SSIM(x, y))
// SSIM (Wang et al. 2004) with an 11x11 Gaussian window (sigma 1.5), C1 = 0.01^2, C2 = 0.03^2,
// zero padding ("same"), averaged over every pixel and channel: the loss of the 3DGS trainers
// the reference runs (LAMBDA_DSSIM 0.2, phase2/logs/run_4559238/runs/b_room_up_s10/
// training_config.yaml:100), computed there by the fused-ssim extension (fusedssimCUDA /
// fusedssim_backwardCUDA, results/phase1/README.md:46-47).
//
// One workgroup per 16x16 tile and channel. Forward: the tile plus a 5-pixel halo of both
// images goes to LDS, the five moments (x, y, x^2, y^2, xy) are filtered separably (rows, then
// columns), and each pixel writes the three partial derivatives of its SSIM value the backward
// needs (dS/dmu_x, dS/dE[x^2], dS/dE[xy]) plus per-workgroup partial sums for the loss value.
// Backward: the same separable filter on the three partial maps (the Gaussian is symmetric, so
// the transpose of the zero-padded filter is itself), then
//   dL/dx = (1 - lambda) sign(x - y) / N - lambda / N (G*a + 2 x G*b + y G*c).
#include <mutex>

#include "gs_host.h"

namespace gs {

constexpr int kSsTile = 16;
constexpr int kSsHalo = 5;
constexpr int kSsIn = kSsTile + 2 * kSsHalo;  // 26
constexpr float kSsC1 = 0.01f * 0.01f;
constexpr float kSsC2 = 0.03f * 0.03f;

struct SsimWeights {
  float w[11];
};

// Loads a kSsIn x kSsIn patch (zero outside the image) of plane `src` at tile (tx, ty).
__device__ __forceinline__ void load_patch(const float* __restrict__ src, int H, int W, int tx, int ty,
                                           float (*dst)[kSsIn]) {
  for (int k = threadIdx.x; k < kSsIn * kSsIn; k += 256) {
    const int r = k / kSsIn, c = k - r * kSsIn;
    const int py = ty * kSsTile + r - kSsHalo, px = tx * kSsTile + c - kSsHalo;
    dst[r][c] = (py >= 0 && py < H && px >= 0 && px < W) ? src[static_cast<int64_t>(py) * W + px] : 0.0f;
  }
}

__global__ __launch_bounds__(256) void ssim_fwd_kernel(const float* __restrict__ img, const float* __restrict__ gt,
                                                       int H, int W, SsimWeights G, float* __restrict__ dmap,
                                                       float* __restrict__ partials) {
  __shared__ float s_x[kSsIn][kSsIn], s_y[kSsIn][kSsIn];
  __shared__ float s_h[5][kSsIn][kSsTile];  // row-filtered x, y, xx, yy, xy
  __shared__ float s_red[2][4];
  const int tx = blockIdx.x, ty = blockIdx.y, ch = blockIdx.z;
  const int64_t plane = static_cast<int64_t>(H) * W;
  const float* xp = img + ch * plane;
  const float* yp = gt + ch * plane;
  load_patch(xp, H, W, tx, ty, s_x);
  load_patch(yp, H, W, tx, ty, s_y);
  __syncthreads();
  // rows: 26 x 16 outputs, 5 moments each
  for (int k = threadIdx.x; k < kSsIn * kSsTile; k += 256) {
    const int r = k / kSsTile, c = k - r * kSsTile;
    float mx = 0.0f, my = 0.0f, mxx = 0.0f, myy = 0.0f, mxy = 0.0f;
#pragma unroll
    for (int t = 0; t < 11; ++t) {
      const float a = s_x[r][c + t], b = s_y[r][c + t], w = G.w[t];
      mx = fmaf(w, a, mx);
      my = fmaf(w, b, my);
      mxx = fmaf(w, a * a, mxx);
      myy = fmaf(w, b * b, myy);
      mxy = fmaf(w, a * b, mxy);
    }
    s_h[0][r][c] = mx;
    s_h[1][r][c] = my;
    s_h[2][r][c] = mxx;
    s_h[3][r][c] = myy;
    s_h[4][r][c] = mxy;
  }
  __syncthreads();
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
  float m[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 11; ++t) {
    const float w = G.w[t];
#pragma unroll
    for (int q = 0; q < 5; ++q) m[q] = fmaf(w, s_h[q][r + t][c], m[q]);
  }
  const int py = ty * kSsTile + r, px = tx * kSsTile + c;
  const bool inside = py < H && px < W;
  float s_val = 0.0f, l1 = 0.0f;
  if (inside) {
    const float mu1 = m[0], mu2 = m[1];
    const float s11 = m[2] - mu1 * mu1, s22 = m[3] - mu2 * mu2, s12 = m[4] - mu1 * mu2;
    const float A = 2.0f * mu1 * mu2 + kSsC1, B = 2.0f * s12 + kSsC2;
    const float Cc = mu1 * mu1 + mu2 * mu2 + kSsC1, D = s11 + s22 + kSsC2;
    const float S = (A * B) / (Cc * D);
    s_val = S;
    const float xv = s_x[r + kSsHalo][c + kSsHalo], yv = s_y[r + kSsHalo][c + kSsHalo];
    l1 = fabsf(xv - yv);
    if (dmap) {
      const int64_t p = static_cast<int64_t>(py) * W + px;
      const float dmu = S * (2.0f * mu2 / A - 2.0f * mu2 / B - 2.0f * mu1 / Cc + 2.0f * mu1 / D);
      dmap[(ch * 3 + 0) * plane + p] = dmu;                        // dS/dmu_x
      dmap[(ch * 3 + 1) * plane + p] = -S / D;                     // dS/dE[x^2]
      dmap[(ch * 3 + 2) * plane + p] = 2.0f * S / B;               // dS/dE[xy]
    }
  }
  // workgroup sums of S and |x - y| (fixed order: deterministic)
  float a0 = s_val, a1 = l1;
  for (int o = 32; o > 0; o >>= 1) {
    a0 += __shfl_xor(a0, o, 64);
    a1 += __shfl_xor(a1, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    s_red[0][threadIdx.x >> 6] = a0;
    s_red[1][threadIdx.x >> 6] = a1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t b = (static_cast<int64_t>(ch) * gridDim.y + ty) * gridDim.x + tx;
    partials[2 * b] = (s_red[0][0] + s_red[0][1]) + (s_red[0][2] + s_red[0][3]);
    partials[2 * b + 1] = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);
  }
}

// One workgroup: sums the per-tile partials in double, writes loss[0] = total, loss[1] = mean
// |x - y|, loss[2] = mean SSIM.
__global__ __launch_bounds__(256) void ssim_reduce_kernel(const float* __restrict__ partials, int64_t n_blocks,
                                                          double n_elems, float lambda, float* __restrict__ loss) {
  __shared__ double s_sum[2][256];
  double a = 0.0, b = 0.0;
  for (int64_t k = threadIdx.x; k < n_blocks; k += 256) {
    a += partials[2 * k];
    b += partials[2 * k + 1];
  }
  s_sum[0][threadIdx.x] = a;
  s_sum[1][threadIdx.x] = b;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (static_cast<int>(threadIdx.x) < s) {
      s_sum[0][threadIdx.x] += s_sum[0][threadIdx.x + s];
      s_sum[1][threadIdx.x] += s_sum[1][threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double ssim = s_sum[0][0] / n_elems, l1 = s_sum[1][0] / n_elems;
    loss[0] = static_cast<float>((1.0 - lambda) * l1 + lambda * (1.0 - ssim));
    loss[1] = static_cast<float>(l1);
    loss[2] = static_cast<float>(ssim);
  }
}

__global__ __launch_bounds__(256) void ssim_bwd_kernel(const float* __restrict__ img, const float* __restrict__ gt,
                                                       const float* __restrict__ dmap, int H, int W, SsimWeights G,
                                                       float k_l1, float k_ssim, const float* __restrict__ dloss,
                                                       float* __restrict__ grad) {
  __shared__ float s_d[3][kSsIn][kSsIn];
  __shared__ float s_h[3][kSsIn][kSsTile];
  const int tx = blockIdx.x, ty = blockIdx.y, ch = blockIdx.z;
  const int64_t plane = static_cast<int64_t>(H) * W;
  for (int q = 0; q < 3; ++q) load_patch(dmap + (ch * 3 + q) * plane, H, W, tx, ty, s_d[q]);
  __syncthreads();
  for (int k = threadIdx.x; k < kSsIn * kSsTile; k += 256) {
    const int r = k / kSsTile, c = k - r * kSsTile;
    float h0 = 0.0f, h1 = 0.0f, h2 = 0.0f;
#pragma unroll
    for (int t = 0; t < 11; ++t) {
      const float w = G.w[t];
      h0 = fmaf(w, s_d[0][r][c + t], h0);
      h1 = fmaf(w, s_d[1][r][c + t], h1);
      h2 = fmaf(w, s_d[2][r][c + t], h2);
    }
    s_h[0][r][c] = h0;
    s_h[1][r][c] = h1;
    s_h[2][r][c] = h2;
  }
  __syncthreads();
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
  const int py = ty * kSsTile + r, px = tx * kSsTile + c;
  if (py >= H || px >= W) return;
  float ga = 0.0f, gb = 0.0f, gc = 0.0f;
#pragma unroll
  for (int t = 0; t < 11; ++t) {
    const float w = G.w[t];
    ga = fmaf(w, s_h[0][r + t][c], ga);
    gb = fmaf(w, s_h[1][r + t][c], gb);
    gc = fmaf(w, s_h[2][r + t][c], gc);
  }
  const int64_t p = ch * plane + static_cast<int64_t>(py) * W + px;
  const float x = img[p], y = gt[p];
  const float sgn = x > y ? 1.0f : (x < y ? -1.0f : 0.0f);
  const float dS = ga + 2.0f * x * gb + y * gc;
  const float scale = dloss ? dloss[0] : 1.0f;
  grad[p] = scale * (k_l1 * sgn - k_ssim * dS);
}

static SsimWeights ssim_weights() {
  SsimWeights g;
  double w[11], s = 0.0;
  for (int i = 0; i < 11; ++i) {
    const double d = i - 5;
    w[i] = exp(-(d * d) / (2.0 * 1.5 * 1.5));
    s += w[i];
  }
  for (int i = 0; i < 11; ++i) g.w[i] = static_cast<float>(w[i] / s);
  return g;
}

}  // namespace gs

using namespace gs;

static int64_t ssim_blocks(int C, int H, int W) {
  return static_cast<int64_t>((W + kSsTile - 1) / kSsTile) * ((H + kSsTile - 1) / kSsTile) * C;
}

extern "C" size_t gs_l1_ssim_workspace_size(int channels, int height, int width) {
  if (channels <= 0 || height <= 0 || width <= 0) return 0;
  return static_cast<size_t>(ssim_blocks(channels, height, width)) * 2 * sizeof(float);
}

// Both forward entry points: the per-tile partial sums go to `partials` (2 floats per tile and
// channel, every one written by ssim_fwd_kernel before ssim_reduce_kernel reads it, so nothing
// has to start at zero).
static int l1_ssim_fwd_launch(const float* image, const float* target, int channels, int height, int width,
                              float lambda_dssim, float* dmap, float* loss, float* partials, hipStream_t st) {
  const dim3 grid((width + kSsTile - 1) / kSsTile, (height + kSsTile - 1) / kSsTile, channels);
  hipLaunchKernelGGL(ssim_fwd_kernel, grid, dim3(256), 0, st, image, target, height, width, ssim_weights(), dmap,
                     partials);
  const double n = static_cast<double>(channels) * height * width;
  hipLaunchKernelGGL(ssim_reduce_kernel, dim3(1), dim3(256), 0, st, partials, ssim_blocks(channels, height, width),
                     n, lambda_dssim, loss);
  return check_launch("l1_ssim_fwd");
}

static int l1_ssim_check_args(const float* image, const float* target, int channels, int height, int width,
                              float lambda_dssim, const float* loss) {
  GS_REQUIRE(channels > 0 && channels <= 65535 && height > 0 && width > 0, GS_ERR_ARG, "invalid image size");
  GS_REQUIRE(image && target && loss, GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(lambda_dssim >= 0.0f && lambda_dssim <= 1.0f, GS_ERR_ARG, "lambda_dssim must be in [0, 1]");
  return GS_OK;
}

extern "C" int gs_l1_ssim_fwd(const float* image, const float* target, int channels, int height, int width,
                              float lambda_dssim, float* dmap, float* loss, void* workspace, size_t workspace_bytes,
                              void* stream) {
  clear_error();
  const int rc = l1_ssim_check_args(image, target, channels, height, width, lambda_dssim, loss);
  if (rc != GS_OK) return rc;
  const size_t need = gs_l1_ssim_workspace_size(channels, height, width);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  return l1_ssim_fwd_launch(image, target, channels, height, width, lambda_dssim, dmap, loss,
                            static_cast<float*>(workspace), as_stream(stream));
}

// ---------------------------------------------------------------------------------------------
// Allocation-free forward: the partial sums live in a static device array of the library (one
// copy per GPU, held until the process ends). Host code never passes `scratch` itself (in host
// code that name is a stand-in, not a device address): each device's address is looked up once
// with hipGetSymbolAddress while that device is current, and kept per device.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) float scratch[2 * GS_L1_SSIM_NOALLOC_MAX_TILES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static float* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (NULL and an error message on failure).
static float* scratch_on_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("l1_ssim_fwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_error("l1_ssim_fwd_noalloc: device %d beyond the %d the library keeps scratch addresses for", dev,
              kMaxScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    float* p = nullptr;
    e = hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("l1_ssim_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

extern "C" int gs_l1_ssim_fwd_noalloc(const float* image, const float* target, int channels, int height, int width,
                                      float lambda_dssim, float* dmap, float* loss, void* stream) {
  clear_error();
  const int rc = l1_ssim_check_args(image, target, channels, height, width, lambda_dssim, loss);
  if (rc != GS_OK) return rc;
  const int64_t tiles = ssim_blocks(channels, height, width);
  GS_REQUIRE(tiles <= GS_L1_SSIM_NOALLOC_MAX_TILES, GS_ERR_ARG,
             "l1_ssim_fwd_noalloc: %d x %d x %d images have %lld tiles x channels, more than the %d its static "
             "buffer holds (use gs_l1_ssim_fwd with a workspace)",
             channels, height, width, static_cast<long long>(tiles), GS_L1_SSIM_NOALLOC_MAX_TILES);
  float* partials = scratch_on_current_device();
  if (partials == nullptr) return GS_ERR_LAUNCH;
  return l1_ssim_fwd_launch(image, target, channels, height, width, lambda_dssim, dmap, loss, partials,
                            as_stream(stream));
}

extern "C" int gs_l1_ssim_bwd(const float* image, const float* target, const float* dmap, int channels, int height,
                              int width, float lambda_dssim, const float* grad_loss, float* grad_image, void* stream) {
  clear_error();
  GS_REQUIRE(channels > 0 && channels <= 65535 && height > 0 && width > 0, GS_ERR_ARG, "invalid image size");
  GS_REQUIRE(image && target && dmap && grad_image, GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(lambda_dssim >= 0.0f && lambda_dssim <= 1.0f, GS_ERR_ARG, "lambda_dssim must be in [0, 1]");
  const double n = static_cast<double>(channels) * height * width;
  const dim3 grid((width + kSsTile - 1) / kSsTile, (height + kSsTile - 1) / kSsTile, channels);
  hipLaunchKernelGGL(ssim_bwd_kernel, grid, dim3(256), 0, as_stream(stream), image, target, dmap, height, width,
                     ssim_weights(), static_cast<float>((1.0 - lambda_dssim) / n), static_cast<float>(lambda_dssim / n),
                     grad_loss, grad_image);
  return check_launch("l1_ssim_bwd");
}
