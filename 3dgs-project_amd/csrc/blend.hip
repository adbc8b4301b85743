// 3D alpha blending: forward (one 16x16 tile per 256-lane workgroup) and the bucketed
// backward (one wavefront per 32-entry bucket, each lane owning 4 pixels).
//
// Pixel layout inside a tile: thread t owns pixel (t % 16, t / 16), so wavefront w owns
// rows 4w .. 4w+3 (a 16x4 "strip"). A splat is evaluated for a strip only if its pixel
// bounds overlap the strip's rows; the forward, the backward and the CPU oracle apply this
// rule identically, so the backward replays exactly the forward's splat sequence (the same
// purpose as Faster-GS's per-subtile culling, phase1/fastergs_macro.patch:92-104).
#include "gs_host.h"

namespace gs {

// log2-domain exponent of the Gaussian at offset (dx, dy) = mean - pixel centre, with the
// conic pre-scaled by (-1/2 log2 e, -log2 e, -1/2 log2 e). Clamped at 0.
__device__ __forceinline__ float power2(float qa, float qb, float qc, float dx, float dy) {
  float t = qb * dy;
  t = fmaf(qa, dx, t);
  float u = qc * dy;
  u = u * dy;
  const float e = fmaf(dx, t, u);
  return fminf(e, 0.0f);
}

__device__ __forceinline__ uint32_t strip_mask(const int4 d, int tile_y0) {
  uint32_t m = 0;
#pragma unroll
  for (int s = 0; s < kStrips; ++s) {
    const int r0 = tile_y0 + kStripRows * s, r1 = r0 + kStripRows - 1;
    if (d.z <= r1 && d.w >= r0) m |= 1u << s;
  }
  return m;
}

// ---------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kTilePixels) void blend_fwd_3d_kernel(
    const SplatRec* __restrict__ rec, const uint2* __restrict__ ranges,
    const uint32_t* __restrict__ point_list, const uint32_t* __restrict__ bucket_offsets, int W,
    int H, int tiles_x, float bg_r, float bg_g, float bg_b, float* __restrict__ image,
    float* __restrict__ final_T, int32_t* __restrict__ n_contrib, uint32_t* __restrict__ tile_max,
    float4* __restrict__ ckpt) {
  __shared__ float4 s_p0[kTilePixels];  // mx, my, qa, qb
  __shared__ float4 s_p1[kTilePixels];  // qc, o, r, g
  __shared__ float2 s_p2[kTilePixels];  // b, strip mask
  __shared__ uint32_t s_max;

  const int tile = blockIdx.x;
  const int tx = tile % tiles_x, ty = tile / tiles_x;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int px = tx * kTile + (t & 15), py = ty * kTile + (t >> 4);
  const bool inside = px < W && py < H;
  const float pxf = static_cast<float>(px) + 0.5f, pyf = static_cast<float>(py) + 0.5f;
  const uint2 range = ranges[tile];
  const int len = static_cast<int>(range.y - range.x);
  float4* ck = ckpt + static_cast<int64_t>(bucket_offsets[tile]) * kTilePixels + t;
  if (t == 0) s_max = 0;

  float T = 1.0f, Cr = 0.0f, Cg = 0.0f, Cb = 0.0f;
  int last = 0;
  bool done = !inside;
  for (int b0 = 0; b0 < len; b0 += kTilePixels) {
    if (__syncthreads_count(done ? 1 : 0) == kTilePixels) break;
    const int j = b0 + t;
    if (j < len) {
      const uint32_t g = point_list[range.x + j];
      const SplatRec r = rec[g];
      s_p0[t] = make_float4(r.a.x, r.a.y, r.a.z * kNegHalfLog2e, r.a.w * kNegLog2e);
      s_p1[t] = make_float4(r.b.x * kNegHalfLog2e, r.b.y, r.c.x, r.c.y);
      s_p2[t] = make_float2(r.c.z, __uint_as_float(strip_mask(r.d, ty * kTile)));
    }
    __syncthreads();
    const int nb = min(kTilePixels, len - b0);
    for (int jj = 0; jj < nb; ++jj) {
      const int idx = b0 + jj;
      if ((idx & (kBucket - 1)) == 0) ck[static_cast<int64_t>(idx / kBucket) * kTilePixels] = make_float4(Cr, Cg, Cb, T);
      if (done) continue;
      const float2 p2 = s_p2[jj];
      if (((__float_as_uint(p2.y) >> wave) & 1u) == 0u) continue;  // wave-uniform
      const float4 p0 = s_p0[jj];
      const float4 p1 = s_p1[jj];
      const float dx = p0.x - pxf, dy = p0.y - pyf;
      const float G = exp2_neg(power2(p0.z, p0.w, p1.x, dx, dy));
      const float alpha = p1.y * G;
      if (alpha < kAlphaMin) continue;
      const float w = alpha * T;
      Cr = fmaf(p1.z, w, Cr);
      Cg = fmaf(p1.w, w, Cg);
      Cb = fmaf(p2.x, w, Cb);
      T = T * (1.0f - alpha);
      last = idx + 1;
      if (T < kTStop) done = true;
    }
  }
  if (inside) {
    const int64_t pix = static_cast<int64_t>(py) * W + px;
    const int64_t HW = static_cast<int64_t>(H) * W;
    image[pix] = fmaf(T, bg_r, Cr);
    image[HW + pix] = fmaf(T, bg_g, Cg);
    image[2 * HW + pix] = fmaf(T, bg_b, Cb);
    final_T[pix] = T;
    n_contrib[pix] = last;
    if (last > 0) atomicMax(&s_max, static_cast<uint32_t>(last));
  }
  __syncthreads();
  if (t == 0) tile_max[tile] = s_max;
}

// ---------------------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------------------

// Sum over the wavefront; the result is returned to every lane (via lane 63 and a
// readlane). Row reductions use DPP row shifts, rows are combined with row_bcast.
__device__ __forceinline__ float wave_sum(float v) {
  int x = __float_as_int(v);
  float s = v;
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true));   // row_shr:1
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true));   // row_shr:2
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x113, 0xf, 0xf, true));   // row_shr:3
  x = __float_as_int(s);
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xe, false));  // row_shr:4
  x = __float_as_int(s);
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xc, false));  // row_shr:8
  x = __float_as_int(s);
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));  // row_bcast:15
  x = __float_as_int(s);
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 63));
}

constexpr int kBwdWaves = 4;

__global__ __launch_bounds__(kBwdWaves * kWave) void blend_bwd_3d_kernel(
    const SplatRec* __restrict__ rec, const uint2* __restrict__ ranges,
    const uint32_t* __restrict__ point_list, const uint32_t* __restrict__ bucket_offsets,
    const uint32_t* __restrict__ bucket_to_tile, int n_tiles, int W, int H, int tiles_x,
    const float* __restrict__ image, const float* __restrict__ grad_image,
    const float* __restrict__ final_T, const float* __restrict__ grad_alpha,
    const int32_t* __restrict__ n_contrib, const uint32_t* __restrict__ tile_max,
    const float4* __restrict__ ckpt, float* __restrict__ grad2d) {
  __shared__ float4 s_p0[kBwdWaves][kBucket];  // mx, my, qa, qb
  __shared__ float4 s_p1[kBwdWaves][kBucket];  // qc, o, A, B
  __shared__ float4 s_p2[kBwdWaves][kBucket];  // C, r, g, b
  __shared__ uint32_t s_m[kBwdWaves][kBucket];  // strip mask
  __shared__ uint32_t s_id[kBwdWaves][kBucket];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kBwdWaves + wave;
  const uint32_t n_buckets = bucket_offsets[n_tiles];
  if (b >= n_buckets) return;  // whole wavefront
  const uint32_t tile = bucket_to_tile[b];
  const int bstart = static_cast<int>(b - bucket_offsets[tile]) * kBucket;
  const int tmax = static_cast<int>(tile_max[tile]);
  if (bstart >= tmax) return;
  const int bsize = min(kBucket, tmax - bstart);
  const uint2 range = ranges[tile];
  const int tx = static_cast<int>(tile) % tiles_x, ty = static_cast<int>(tile) / tiles_x;

  if (lane < bsize) {
    const uint32_t g = point_list[range.x + bstart + lane];
    const SplatRec r = rec[g];
    s_p0[wave][lane] = make_float4(r.a.x, r.a.y, r.a.z * kNegHalfLog2e, r.a.w * kNegLog2e);
    s_p1[wave][lane] = make_float4(r.b.x * kNegHalfLog2e, r.b.y, r.a.z, r.a.w);
    s_p2[wave][lane] = make_float4(r.b.x, r.c.x, r.c.y, r.c.z);
    s_m[wave][lane] = strip_mask(r.d, ty * kTile);
    s_id[wave][lane] = g;
  }

  // per-pixel state: pixel p = 64 r + lane, row 4 r + lane / 16, column lane % 16
  const int64_t HW = static_cast<int64_t>(H) * W;
  const int px = tx * kTile + (lane & 15);
  const float pxf = static_cast<float>(px) + 0.5f;
  float T[kPixPerLane], rho[kPixPerLane], Gr[kPixPerLane], Gg[kPixPerLane], Gb[kPixPerLane];
  float pyf[kPixPerLane];
  int lim[kPixPerLane];
#pragma unroll
  for (int r = 0; r < kPixPerLane; ++r) {
    const int py = ty * kTile + kStripRows * r + (lane >> 4);
    pyf[r] = static_cast<float>(py) + 0.5f;
    T[r] = 0.0f;
    rho[r] = 0.0f;
    Gr[r] = Gg[r] = Gb[r] = 0.0f;
    lim[r] = 0;
    if (px < W && py < H) {
      const int64_t pix = static_cast<int64_t>(py) * W + px;
      const int used = n_contrib[pix] - bstart;
      if (used > 0) {
        lim[r] = used;
        Gr[r] = grad_image[pix];
        Gg[r] = grad_image[HW + pix];
        Gb[r] = grad_image[2 * HW + pix];
        const float4 c = ckpt[b * kTilePixels + kWave * r + lane];
        T[r] = c.w;
        rho[r] = Gr[r] * (image[pix] - c.x) + Gg[r] * (image[HW + pix] - c.y) +
                 Gb[r] * (image[2 * HW + pix] - c.z);
        // alpha = 1 - T_final output: its gradient enters like a background term
        if (grad_alpha) rho[r] -= grad_alpha[pix] * final_T[pix];
      }
    }
  }
  wave_sync();

  for (int j = 0; j < bsize; ++j) {
    const uint32_t m = s_m[wave][j];
    const float4 p0 = s_p0[wave][j];
    const float4 p1 = s_p1[wave][j];
    const float4 p2 = s_p2[wave][j];
    float acc[11];
#pragma unroll
    for (int k = 0; k < 11; ++k) acc[k] = 0.0f;
    bool used = false;
#pragma unroll
    for (int r = 0; r < kPixPerLane; ++r) {
      if (((m >> r) & 1u) == 0u) continue;  // wave-uniform
      if (j >= lim[r]) continue;
      const float dx = p0.x - pxf, dy = p0.y - pyf[r];
      const float G = exp2_neg(power2(p0.z, p0.w, p1.x, dx, dy));
      const float alpha = p1.y * G;
      if (alpha < kAlphaMin) continue;
      used = true;
      const float w = T[r] * alpha;
      const float dot = Gr[r] * p2.y + Gg[r] * p2.z + Gb[r] * p2.w;
      acc[6] += w * Gr[r];
      acc[7] += w * Gg[r];
      acc[8] += w * Gb[r];
      rho[r] = fmaf(-w, dot, rho[r]);
      const float oma = 1.0f - alpha;
      const float dLda = T[r] * dot - rho[r] * __builtin_amdgcn_rcpf(fmaxf(oma, kOneMinusAlphaEps));
      acc[5] += G * dLda;
      const float hp = alpha * dLda;  // dL/dpower (natural)
      acc[2] += -0.5f * hp * dx * dx;
      acc[3] += -hp * dx * dy;
      acc[4] += -0.5f * hp * dy * dy;
      const float gmx = -hp * (p1.z * dx + p1.w * dy);
      const float gmy = -hp * (p1.w * dx + p2.x * dy);
      acc[0] += gmx;
      acc[1] += gmy;
      acc[9] += fabsf(gmx);
      acc[10] += fabsf(gmy);
      T[r] = T[r] * oma;
    }
    if (__ballot(used ? 1 : 0) == 0) continue;  // wave-uniform
    float mine = 0.0f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const float s = wave_sum(acc[k]);
      mine = (lane == k) ? s : mine;
    }
    if (lane < 11) unsafeAtomicAdd(grad2d + static_cast<int64_t>(s_id[wave][j]) * kGrad2D + lane, mine);
  }
}

}  // namespace gs

using namespace gs;

extern "C" int gs_blend_fwd_3d(const float* splat_rec, const uint32_t* ranges,
                               const uint32_t* point_list, const uint32_t* bucket_offsets,
                               int width, int height, const float* bg, float* image,
                               float* final_T, int32_t* n_contrib, uint32_t* tile_max,
                               float* ckpt, void* stream) {
  clear_error();
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARG, "image size must be positive");
  // splat_rec, point_list and ckpt may be NULL when the scene has no instances
  GS_REQUIRE(ranges && bucket_offsets && image && final_T && n_contrib && tile_max, GS_ERR_ARG,
             "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16) && aligned(ckpt, 16) && aligned(ranges, 8), GS_ERR_ALIGN,
             "splat_rec/ckpt must be 16-byte and ranges 8-byte aligned");
  const int tiles_x = (width + kTile - 1) / kTile, tiles_y = (height + kTile - 1) / kTile;
  const float br = bg ? bg[0] : 0.0f, bgg = bg ? bg[1] : 0.0f, bb = bg ? bg[2] : 0.0f;
  hipLaunchKernelGGL(blend_fwd_3d_kernel, dim3(tiles_x * tiles_y), dim3(kTilePixels), 0,
                     as_stream(stream), reinterpret_cast<const SplatRec*>(splat_rec),
                     reinterpret_cast<const uint2*>(ranges), point_list, bucket_offsets, width,
                     height, tiles_x, br, bgg, bb, image, final_T, n_contrib, tile_max,
                     reinterpret_cast<float4*>(ckpt));
  return check_launch("blend_fwd_3d");
}

extern "C" int gs_blend_bwd_3d(const float* splat_rec, const uint32_t* ranges,
                               const uint32_t* point_list, const uint32_t* bucket_offsets,
                               const uint32_t* bucket_to_tile, int64_t n_buckets_max, int64_t n,
                               int width, int height, const float* image, const float* grad_image,
                               const float* final_T, const float* grad_alpha,
                               const int32_t* n_contrib, const uint32_t* tile_max,
                               const float* ckpt, float* grad2d, void* stream) {
  clear_error();
  GS_REQUIRE(width > 0 && height > 0 && n >= 0 && n_buckets_max >= 0, GS_ERR_ARG,
             "invalid sizes");
  GS_REQUIRE(grad2d || n == 0, GS_ERR_ARG, "null grad2d");
  hipStream_t st = as_stream(stream);
  fill_zero_f32(grad2d, n * kGrad2D, st);
  if (int e = check_launch("blend_bwd_3d (zero fill)")) return e;
  if (n_buckets_max == 0 || n == 0) return GS_OK;
  // splat_rec, point_list and ckpt may be NULL when there are no instances (no bucket reads them)
  GS_REQUIRE(ranges && bucket_offsets && bucket_to_tile && image && grad_image && n_contrib &&
                 tile_max && (final_T || !grad_alpha),
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16) && aligned(ckpt, 16) && aligned(ranges, 8), GS_ERR_ALIGN,
             "splat_rec/ckpt must be 16-byte and ranges 8-byte aligned");
  const int tiles_x = (width + kTile - 1) / kTile, tiles_y = (height + kTile - 1) / kTile;
  const int64_t blocks = (n_buckets_max + kBwdWaves - 1) / kBwdWaves;
  hipLaunchKernelGGL(blend_bwd_3d_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(kBwdWaves * kWave), 0, st, reinterpret_cast<const SplatRec*>(splat_rec),
                     reinterpret_cast<const uint2*>(ranges), point_list, bucket_offsets,
                     bucket_to_tile, tiles_x * tiles_y, width, height, tiles_x, image, grad_image,
                     final_T, grad_alpha, n_contrib, tile_max, reinterpret_cast<const float4*>(ckpt), grad2d);
  return check_launch("blend_bwd_3d");
}
