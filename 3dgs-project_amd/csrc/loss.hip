// Fused L1 + D-SSIM training loss, forward and backward, on [C, H, W] float32 images:
//   L = (1 - lambda) mean|x - y| + lambda (1 - mean SSIM(x, y))
// SSIM (Wang et al. 2004) with an 11x11 Gaussian window (sigma 1.5), C1 = 0.01^2, C2 = 0.03^2,
// zero padding ("same"), averaged over every pixel and channel: the loss of the 3DGS trainers
// the reference runs (LAMBDA_DSSIM 0.2, phase2/logs/run_4559238/runs/b_room_up_s10/
// training_config.yaml:100), computed there by the fused-ssim extension (fusedssimCUDA /
// fusedssim_backwardCUDA, results/phase1/README.md:46-47).
//
// One workgroup per 32x32 tile and channel. Forward: the tile plus a 5-pixel halo of both
// images goes to LDS, the five moments (x, y, x^2, y^2, xy) are filtered separably (rows, then
// columns; in each pass a thread computes four adjacent outputs from the 14 inputs they share,
// so every input is read and squared once), and each pixel writes the three partial derivatives
// of its SSIM value the backward needs (dS/dmu_x, dS/dE[x^2], dS/dE[xy]) plus per-workgroup
// partial sums for the loss value.
// Backward: the same separable filter on the three partial maps (the Gaussian is symmetric, so
// the transpose of the zero-padded filter is itself), then
//   dL/dx = (1 - lambda) sign(x - y) / N - lambda / N (G*a + 2 x G*b + y G*c).
#include <climits>
#include <mutex>

#include "gs_host.h"

namespace gs {

constexpr int kSsTile = 32;                       // output tile side
constexpr int kSsHalo = 5;                        // filter radius
constexpr int kSsIn = kSsTile + 2 * kSsHalo;      // 42: input patch side
constexpr int kSsInS = kSsIn + 2;                 // 44: patch row stride (16-byte rows)
constexpr int kSsHS = kSsTile + 8;                // 40: row stride of the row-filtered planes
constexpr int kSsQ = 4;                           // outputs per thread in each pass
constexpr int kSsGroups = kSsTile / kSsQ;         // 8 column groups (row pass), row groups (column pass)
constexpr int kSsThreads = 256;
constexpr int kSsTaps = 2 * kSsHalo + 1;          // 11
constexpr int kSsSpan = kSsQ + kSsTaps - 1;       // 14 inputs per thread and pass
constexpr int kSsLimitTile = 16;                  // tile side of the allocation-free entry's size limit
constexpr float kSsC1 = 0.01f * 0.01f;
constexpr float kSsC2 = 0.03f * 0.03f;
constexpr int cmax(int a, int b) { return a > b ? a : b; }
// Forward LDS (floats): the five row-filtered planes, with the x and y patches placed after the
// first three, so that only planes 3 and 4 share memory with the patches.
constexpr int kSsFwdHold = 3;  // first plane held in registers over the row pass's barrier
constexpr int kSsFwdXy = kSsFwdHold * kSsIn * kSsHS;
constexpr int kSsFwdLds = cmax(kSsFwdXy + 2 * kSsIn * kSsInS, 5 * kSsIn * kSsHS);
// Backward: the three patches, then (same memory, every plane held) their row-filtered planes.
constexpr int kSsBwdLds = cmax(3 * kSsIn * kSsInS, 3 * kSsIn * kSsHS);
static_assert(kSsGroups * kSsTile == kSsThreads, "column pass: one thread per (column, row group)");
static_assert(kSsHS % 4 == 0 && kSsInS % 4 == 0, "16-byte LDS rows");
static_assert(kSsQ * (kSsGroups - 1) + 4 * ((kSsSpan + 3) / 4) <= kSsInS, "row pass float4 reads stay in a patch row");
static_assert(kSsQ * (kSsGroups - 1) + kSsSpan <= kSsIn, "column pass reads stay inside the filtered rows");

struct SsimWeights {
  float w[11];
};

// Loads the kSsIn x kSsIn patches (zero outside the image) of the NP planes src[p] around tile
// (tx, ty) into rows of kSsInS floats (dst + p * kSsIn * kSsInS; the last two columns of a row
// are not written and not used). Every load of a thread is issued before its first LDS store,
// so a workgroup waits for memory once. With kL1 (NP = 2: x and y) the thread's sum of |x - y|
// over the loaded pixels of the tile itself (not its halo) is added to l1.
template <int NP, bool kL1>
__device__ __forceinline__ void load_patches(const float* const (&src)[NP], int H, int W, int tx, int ty,
                                             float* __restrict__ dst, float& l1) {
  constexpr int kIters = (kSsIn * kSsIn + kSsThreads - 1) / kSsThreads;  // 7
  constexpr int kStepR = kSsThreads / kSsIn, kStepC = kSsThreads % kSsIn;  // 256 = 6 rows + 4
  float v[NP][kIters];
  int at[kIters];
  int r = static_cast<int>(threadIdx.x) / kSsIn, c = static_cast<int>(threadIdx.x) - r * kSsIn;
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    // element k = threadIdx.x + it * kSsThreads of the patch is (r, c)
    const int py = ty * kSsTile + r - kSsHalo, px = tx * kSsTile + c - kSsHalo;
    const bool here = r < kSsIn;
    const bool in = here && py >= 0 && py < H && px >= 0 && px < W;
    const int64_t off = in ? static_cast<int64_t>(py) * W + px : 0;
    at[it] = here ? r * kSsInS + c : -1;
#pragma unroll
    for (int p = 0; p < NP; ++p) v[p][it] = in ? src[p][off] : 0.0f;
    if constexpr (kL1) {
      const bool tile_px = in && r >= kSsHalo && r < kSsHalo + kSsTile && c >= kSsHalo && c < kSsHalo + kSsTile;
      l1 += tile_px ? fabsf(v[0][it] - v[1][it]) : 0.0f;
    }
    r += kStepR;
    c += kStepC;
    if (c >= kSsIn) {
      c -= kSsIn;
      ++r;
    }
  }
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    if (at[it] < 0) continue;
#pragma unroll
    for (int p = 0; p < NP; ++p) dst[p * kSsIn * kSsInS + at[it]] = v[p][it];
  }
}

// Row pass of NP planes of a patch: item (r, g) filters patch row r (0 .. kSsIn-1) at the kSsQ
// output columns kSsQ g .. kSsQ g + 3 from the kSsSpan inputs starting there (read as float4s).
// Every input is read once; with kMoments (NP = 2: x and y) the five moments x, y, x^2, y^2, xy
// are filtered and their products formed once per input. Output planes: [NO][kSsIn][kSsHS]. The
// planes from kHold on may share memory with the patch: they are kept in registers until the
// workgroup has synchronised, then stored; planes below kHold are stored as each item ends. The
// caller synchronises before reading any plane.
template <int NP, bool kMoments, int kHold>
__device__ __forceinline__ void row_pass(const float* s_in, float* s_h, const SsimWeights& G) {
  constexpr int NO = kMoments ? 5 : NP;
  constexpr int kItems = kSsIn * kSsGroups;
  constexpr int kRounds = (kItems + kSsThreads - 1) / kSsThreads;
  float acc[kRounds][kSsQ][NO];
#pragma unroll
  for (int rd = 0; rd < kRounds; ++rd) {
    const int it = static_cast<int>(threadIdx.x) + rd * kSsThreads;
    if (it >= kItems) continue;
    const int r = it / kSsGroups, g = it - r * kSsGroups;
#pragma unroll
    for (int i4 = 0; i4 < (kSsSpan + 3) / 4; ++i4) {
      float v[NP][4];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const float4 f = *reinterpret_cast<const float4*>(s_in + (p * kSsIn + r) * kSsInS + kSsQ * g + 4 * i4);
        v[p][0] = f.x;
        v[p][1] = f.y;
        v[p][2] = f.z;
        v[p][3] = f.w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * i4 + e;  // input column kSsQ g + i
        if (i >= kSsSpan) continue;
        float m[NO];
        if constexpr (kMoments) {
          m[0] = v[0][e];
          m[1] = v[1][e];
          m[2] = v[0][e] * v[0][e];
          m[3] = v[1][e] * v[1][e];
          m[4] = v[0][e] * v[1][e];
        } else {
#pragma unroll
          for (int p = 0; p < NP; ++p) m[p] = v[p][e];
        }
#pragma unroll
        for (int q = 0; q < kSsQ; ++q) {
          const int t = i - q;  // tap of output column kSsQ g + q (taps in increasing order)
          if (t < 0 || t >= kSsTaps) continue;
#pragma unroll
          for (int o = 0; o < NO; ++o)
            acc[rd][q][o] = t == 0 ? G.w[0] * m[o] : fmaf(G.w[t], m[o], acc[rd][q][o]);
        }
      }
    }
#pragma unroll
    for (int o = 0; o < kHold; ++o)
      *reinterpret_cast<float4*>(s_h + (o * kSsIn + r) * kSsHS + kSsQ * g) =
          make_float4(acc[rd][0][o], acc[rd][1][o], acc[rd][2][o], acc[rd][3][o]);
  }
  __syncthreads();  // the patch is read: its memory may now take the held planes
#pragma unroll
  for (int rd = 0; rd < kRounds; ++rd) {
    const int it = static_cast<int>(threadIdx.x) + rd * kSsThreads;
    if (it >= kItems) continue;
    const int r = it / kSsGroups, g = it - r * kSsGroups;
#pragma unroll
    for (int o = kHold; o < NO; ++o)
      *reinterpret_cast<float4*>(s_h + (o * kSsIn + r) * kSsHS + kSsQ * g) =
          make_float4(acc[rd][0][o], acc[rd][1][o], acc[rd][2][o], acc[rd][3][o]);
  }
}

// Column pass: thread (c, g) filters column c of the NO row-filtered planes at the kSsQ output
// rows kSsQ g .. kSsQ g + 3 (acc[q][o]: output row kSsQ g + q, plane o).
template <int NO>
__device__ __forceinline__ void col_pass(const float* __restrict__ s_h, int c, int g, const SsimWeights& G,
                                         float (&acc)[kSsQ][NO]) {
#pragma unroll
  for (int i = 0; i < kSsSpan; ++i) {
    float h[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o) h[o] = s_h[(o * kSsIn + kSsQ * g + i) * kSsHS + c];
#pragma unroll
    for (int q = 0; q < kSsQ; ++q) {
      const int t = i - q;
      if (t < 0 || t >= kSsTaps) continue;
#pragma unroll
      for (int o = 0; o < NO; ++o) acc[q][o] = t == 0 ? G.w[0] * h[o] : fmaf(G.w[t], h[o], acc[q][o]);
    }
  }
}

// The (tile column, tile row, channel) and the linear tile index of this workgroup. The grid is
// one-dimensional over tiles_x * tiles_y * channels tiles in channel-major, row-major order, dealt
// to the XCDs in contiguous bands (xcd_tile), so the tiles around a tile -- which read the same
// halo rows and cache lines -- are mostly in flight in the same L2.
struct SsTile {
  int tx, ty, ch, index;
};
__device__ __forceinline__ SsTile ss_tile(int tiles_x, int tiles_y) {
  SsTile t;
  t.index = xcd_tile(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int per_ch = tiles_x * tiles_y;
  t.ch = t.index / per_ch;
  const int rem = t.index - t.ch * per_ch;
  t.ty = rem / tiles_x;
  t.tx = rem - t.ty * tiles_x;
  return t;
}

// Sum of v over the workgroup (fixed order: deterministic); the result is valid in thread 0.
__device__ __forceinline__ float block_sum(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}

// One workgroup per 32x32 tile and channel.
__global__ __launch_bounds__(kSsThreads) void ssim_fwd_kernel(const float* __restrict__ img,
                                                              const float* __restrict__ gt, int H, int W,
                                                              SsimWeights G, float* __restrict__ dmap,
                                                              float* __restrict__ partials) {
  // row-filtered x, y, xx, yy, xy; the x and y patches from plane kSsFwdHold on
  __shared__ __align__(16) float s_buf[kSsFwdLds];
  __shared__ float s_red[2][4];
  const SsTile tl = ss_tile((W + kSsTile - 1) / kSsTile, (H + kSsTile - 1) / kSsTile);
  const int tx = tl.tx, ty = tl.ty, ch = tl.ch;
  const int64_t plane = static_cast<int64_t>(H) * W;
  const float* const src[2] = {img + ch * plane, gt + ch * plane};
  float l1_sum = 0.0f;
  load_patches<2, true>(src, H, W, tx, ty, s_buf + kSsFwdXy, l1_sum);
  __syncthreads();
  row_pass<2, true, kSsFwdHold>(s_buf + kSsFwdXy, s_buf, G);
  __syncthreads();
  const int c = threadIdx.x & (kSsTile - 1), g = threadIdx.x / kSsTile;
  float m[kSsQ][5];
  col_pass<5>(s_buf, c, g, G, m);
  const int px = tx * kSsTile + c;
  float s_sum = 0.0f;
#pragma unroll
  for (int q = 0; q < kSsQ; ++q) {
    const int oy = kSsQ * g + q;
    const int py = ty * kSsTile + oy;
    if (py >= H || px >= W) continue;
    const float mu1 = m[q][0], mu2 = m[q][1];
    const float mu11 = mu1 * mu1, mu22 = mu2 * mu2, mu12 = mu1 * mu2;
    const float A = 2.0f * mu12 + kSsC1, B = 2.0f * (m[q][4] - mu12) + kSsC2;
    const float Cc = mu11 + mu22 + kSsC1, D = (m[q][2] - mu11) + (m[q][3] - mu22) + kSsC2;
    // Cc >= C1 and D ~ C2 + variances are positive: one reciprocal each, no division
    const float rC = __builtin_amdgcn_rcpf(Cc), rD = __builtin_amdgcn_rcpf(D);
    const float rCD = rC * rD;
    const float S = (A * B) * rCD;
    s_sum += S;
    if (dmap) {
      const int64_t p = static_cast<int64_t>(py) * W + px;
      // dS/dmu_x = S (2 mu2 / A - 2 mu2 / B - 2 mu1 / Cc + 2 mu1 / D)
      //          = 2 mu2 (B - A) / (Cc D) + 2 mu1 S (1 / D - 1 / Cc)
      dmap[(ch * 3 + 0) * plane + p] = 2.0f * (mu2 * ((B - A) * rCD) + mu1 * (S * (rD - rC)));
      dmap[(ch * 3 + 1) * plane + p] = -S * rD;           // dS/dE[x^2] = -S / D
      dmap[(ch * 3 + 2) * plane + p] = 2.0f * (A * rCD);  // dS/dE[xy] = 2 S / B
    }
  }
  const float a0 = block_sum(s_sum, s_red[0]);
  const float a1 = block_sum(l1_sum, s_red[1]);
  if (threadIdx.x == 0) {
    partials[2 * static_cast<int64_t>(tl.index)] = a0;
    partials[2 * static_cast<int64_t>(tl.index) + 1] = a1;
  }
}

// One workgroup of kSsRedThreads: sums the per-tile partials in double (every load of a thread
// issued before its first add), writes loss[0] = total, loss[1] = mean |x - y|, loss[2] = mean
// SSIM.
constexpr int kSsRedThreads = 1024;
constexpr int kSsRedUnroll = 4;
__global__ __launch_bounds__(kSsRedThreads) void ssim_reduce_kernel(const float* __restrict__ partials,
                                                                    int64_t n_blocks, double n_elems, float lambda,
                                                                    float* __restrict__ loss) {
  __shared__ double s_sum[2][kSsRedThreads / 64];
  double a = 0.0, b = 0.0;
  for (int64_t k0 = threadIdx.x; k0 < n_blocks; k0 += kSsRedThreads * kSsRedUnroll) {
    float va[kSsRedUnroll], vb[kSsRedUnroll];
#pragma unroll
    for (int u = 0; u < kSsRedUnroll; ++u) {
      const int64_t k = k0 + static_cast<int64_t>(u) * kSsRedThreads;
      va[u] = k < n_blocks ? partials[2 * k] : 0.0f;
      vb[u] = k < n_blocks ? partials[2 * k + 1] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kSsRedUnroll; ++u) {
      a += static_cast<double>(va[u]);
      b += static_cast<double>(vb[u]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    b += __shfl_xor(b, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    s_sum[0][threadIdx.x >> 6] = a;
    s_sum[1][threadIdx.x >> 6] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double sa = 0.0, sb = 0.0;
    for (int w = 0; w < kSsRedThreads / 64; ++w) {
      sa += s_sum[0][w];
      sb += s_sum[1][w];
    }
    const double ssim = sa / n_elems, l1 = sb / n_elems;
    loss[0] = static_cast<float>((1.0 - lambda) * l1 + lambda * (1.0 - ssim));
    loss[1] = static_cast<float>(l1);
    loss[2] = static_cast<float>(ssim);
  }
}

__global__ __launch_bounds__(kSsThreads) void ssim_bwd_kernel(const float* __restrict__ img,
                                                              const float* __restrict__ gt,
                                                              const float* __restrict__ dmap, int H, int W,
                                                              SsimWeights G, float k_l1, float k_ssim,
                                                              const float* __restrict__ dloss,
                                                              float* __restrict__ grad) {
  // patches of the three partial maps, then (same memory) their row-filtered planes
  __shared__ __align__(16) float s_buf[kSsBwdLds];
  const SsTile tl = ss_tile((W + kSsTile - 1) / kSsTile, (H + kSsTile - 1) / kSsTile);
  const int tx = tl.tx, ty = tl.ty, ch = tl.ch;
  const int64_t plane = static_cast<int64_t>(H) * W;
  // this thread's four pixels of both images, loaded now and used after the filtering
  const int c = threadIdx.x & (kSsTile - 1), g = threadIdx.x / kSsTile;
  const int px = tx * kSsTile + c;
  float xs[kSsQ], ys[kSsQ];
#pragma unroll
  for (int q = 0; q < kSsQ; ++q) {
    const int py = ty * kSsTile + kSsQ * g + q;
    const bool in = py < H && px < W;
    const int64_t p = ch * plane + (in ? static_cast<int64_t>(py) * W + px : 0);
    xs[q] = in ? img[p] : 0.0f;
    ys[q] = in ? gt[p] : 0.0f;
  }
  const float* const src[3] = {dmap + ch * 3 * plane, dmap + (ch * 3 + 1) * plane, dmap + (ch * 3 + 2) * plane};
  float unused = 0.0f;
  load_patches<3, false>(src, H, W, tx, ty, s_buf, unused);
  __syncthreads();
  row_pass<3, false, 0>(s_buf, s_buf, G);
  __syncthreads();
  float f[kSsQ][3];
  col_pass<3>(s_buf, c, g, G, f);
  if (px >= W) return;
  const float scale = dloss ? dloss[0] : 1.0f;
#pragma unroll
  for (int q = 0; q < kSsQ; ++q) {
    const int py = ty * kSsTile + kSsQ * g + q;
    if (py >= H) break;
    const int64_t p = ch * plane + static_cast<int64_t>(py) * W + px;
    const float x = xs[q], y = ys[q];
    const float sgn = x > y ? 1.0f : (x < y ? -1.0f : 0.0f);
    const float dS = f[q][0] + 2.0f * x * f[q][1] + y * f[q][2];
    grad[p] = scale * (k_l1 * sgn - k_ssim * dS);
  }
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

// Tiles x channels of a launch (one partial pair each) for tiles of side `side`.
static int64_t ssim_blocks(int C, int H, int W, int side = kSsTile) {
  return static_cast<int64_t>((W + side - 1) / side) * ((H + side - 1) / side) * C;
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
  const dim3 grid(static_cast<unsigned>(ssim_blocks(channels, height, width)));
  hipLaunchKernelGGL(ssim_fwd_kernel, grid, dim3(kSsThreads), 0, st, image, target, height, width, ssim_weights(),
                     dmap, partials);
  const double n = static_cast<double>(channels) * height * width;
  hipLaunchKernelGGL(ssim_reduce_kernel, dim3(1), dim3(kSsRedThreads), 0, st, partials,
                     ssim_blocks(channels, height, width), n, lambda_dssim, loss);
  return check_launch("l1_ssim_fwd");
}

static int l1_ssim_check_args(const float* image, const float* target, int channels, int height, int width,
                              float lambda_dssim, const float* loss) {
  GS_REQUIRE(channels > 0 && channels <= 65535 && height > 0 && width > 0, GS_ERR_ARG, "invalid image size");
  GS_REQUIRE(ssim_blocks(channels, height, width) <= INT_MAX, GS_ERR_ARG, "image too large (tiles x channels)");
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
  // the limit counts 16-pixel tiles (the kernels' 32-pixel tiles need at most a quarter of them)
  const int64_t tiles = ssim_blocks(channels, height, width, kSsLimitTile);
  static_assert(kSsTile % kSsLimitTile == 0, "a launch needs no more partial pairs than the limit's tiles");
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
  GS_REQUIRE(ssim_blocks(channels, height, width) <= INT_MAX, GS_ERR_ARG, "image too large (tiles x channels)");
  GS_REQUIRE(image && target && dmap && grad_image, GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(lambda_dssim >= 0.0f && lambda_dssim <= 1.0f, GS_ERR_ARG, "lambda_dssim must be in [0, 1]");
  const double n = static_cast<double>(channels) * height * width;
  const dim3 grid(static_cast<unsigned>(ssim_blocks(channels, height, width)));
  hipLaunchKernelGGL(ssim_bwd_kernel, grid, dim3(kSsThreads), 0, as_stream(stream), image, target, dmap, height, width,
                     ssim_weights(), static_cast<float>((1.0 - lambda_dssim) / n), static_cast<float>(lambda_dssim / n),
                     grad_loss, grad_image);
  return check_launch("l1_ssim_bwd");
}
