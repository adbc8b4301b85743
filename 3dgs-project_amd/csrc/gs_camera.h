// Camera description shared by the 3D kernels, and the ellipse / tile test used both to count
// a Gaussian's tiles in the preprocess and to emit its instances in the binning. Both callers
// go through band_columns(), so the count and the emitted keys always agree.
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
  int flags;  // GS_CAM_* bits
  // depth sort keys are order keys relative to the near plane's: a visible Gaussian
  // (near < z < far) gets key(z) - dkey0 in [1, dkey_cull), a culled one dkey_cull, so the
  // sort needs only bit_width(dkey_cull) bits (27 for near/far = 0.01/100)
  uint32_t dkey0, dkey_cull;
};

// Tile assignment. A tile row is a horizontal band of pixel-centre rows [Y0, Y1] (the
// tile's rows clipped to the splat's pixel bounds). The alpha >= 1/255 ellipse
// 1/2 d^T Q d <= thr (d = p - mean) meets the band in a convex set whose x-extent [xl, xr] has
// a closed form; the splat touches the tiles that own a pixel column c (inside its bounds)
// with c + 0.5 in [xl, xr]. Cost is O(tile rows) per splat instead of O(tiles).
struct BandSetup {
  float mx, my, A, B, det, tA, vmax, vr, invA;
  bool ok;
};

__device__ __forceinline__ BandSetup band_setup(const float4 a, const float4 b) {
  BandSetup s;
  s.mx = a.x;
  s.my = a.y;
  s.A = a.z;
  s.B = a.w;
  const float C = b.x, thr = b.w;
  const float t2 = thr + thr;
  s.det = fmaf(s.A, C, -(s.B * s.B));
  s.ok = s.det > 0.0f;
  s.tA = t2 * s.A;
  // reciprocals once per splat, so the per-row work below has no division
  const float idet = 1.0f / s.det;
  s.invA = 1.0f / s.A;
  s.vmax = sqrtf(s.tA * idet);  // half height of the ellipse
  // the rightmost point of the ellipse is (ur, vr) relative to the mean
  const float ur = sqrtf((t2 * C) * idet);
  s.vr = -((s.B / C) * ur);
  return s;
}

// Pixel columns [c0, c1] (clipped to [bx0, bx1]) of the ellipse within the row band.
__device__ __forceinline__ bool band_columns(const BandSetup& s, float Y0, float Y1, int bx0, int bx1,
                                             int& c0, int& c1) {
  if (!s.ok) return false;
  const float v0 = fmaxf(Y0 - s.my, -s.vmax);
  const float v1 = fminf(Y1 - s.my, s.vmax);
  if (!(v0 <= v1)) return false;
  // the x-extent of a row v is concave in v: its max / min over the band sit at the clamped
  // rows of the rightmost / leftmost points
  const float vc = fminf(fmaxf(s.vr, v0), v1);
  const float dr = fmaxf(fmaf(-s.det, vc * vc, s.tA), 0.0f);
  const float br = s.B * vc;
  const float xr = s.mx + (sqrtf(dr) - br) * s.invA;
  const float vl = fminf(fmaxf(-s.vr, v0), v1);
  const float dl = fmaxf(fmaf(-s.det, vl * vl, s.tA), 0.0f);
  const float bl = s.B * vl;
  const float xl = s.mx + (-bl - sqrtf(dl)) * s.invA;
  const float f0 = fmaxf(ceilf(xl - 0.5f), static_cast<float>(bx0));
  const float f1 = fminf(floorf(xr - 0.5f), static_cast<float>(bx1));
  if (!(f0 <= f1)) return false;
  c0 = static_cast<int>(f0);
  c1 = static_cast<int>(f1);
  return true;
}

// Tiles [tx0, tx0 + nt) touched in tile row ty (nt = 0 if the row is missed).
__device__ __forceinline__ uint32_t row_tiles(const BandSetup& s, const int4 d, int ty, int& tx0) {
  const int py0 = max(ty * kTile, d.z), py1 = min(ty * kTile + kTile - 1, d.w);
  int c0, c1;
  if (!band_columns(s, static_cast<float>(py0) + 0.5f, static_cast<float>(py1) + 0.5f, d.x, d.y, c0, c1)) {
    tx0 = 0;
    return 0u;
  }
  tx0 = c0 / kTile;
  return static_cast<uint32_t>(c1 / kTile - tx0 + 1);
}

// Touched-tile counts of a wavefront's 64 splats, their tile rows shared out over the lanes:
// the rows of all splats are numbered in lane order, each lane takes one row at a time
// (binary search for its splat in the row prefix), and the row's tiles are added to the
// splat's count in LDS. Every splat costs the wavefront about its number of rows, so neither
// a few tall splats nor lanes with more rows than others leave lanes idle. `vis` lanes give
// their record halves a, b and pixel bounds d; every lane of the wavefront must call it.
// scratch: kCountScratchWords words of LDS owned by the wavefront. Returns the lane's count.
constexpr int kCountScratchWords = 64 * 12 + 64 + 64;

__device__ __forceinline__ uint32_t wave_count_rows(bool vis, const float4 a, const float4 b, const int4 d,
                                                    int lane, uint32_t* scratch) {
  float4* s_set = reinterpret_cast<float4*>(scratch);  // [64][3]: band setup and bounds
  uint32_t* s_rex = scratch + 64 * 12;                  // exclusive prefix of the rows
  uint32_t* s_cnt = s_rex + 64;                         // tiles per splat
  uint32_t rows = 0;
  if (vis) {
    const BandSetup s = band_setup(a, b);
    rows = static_cast<uint32_t>(max(d.w / kTile - d.z / kTile + 1, 0));
    s_set[3 * lane] = make_float4(s.mx, s.my, s.B, s.det);
    s_set[3 * lane + 1] = make_float4(s.tA, s.vmax, s.vr, s.invA);
    s_set[3 * lane + 2] = make_float4(__int_as_float(d.x), __int_as_float(d.y), __int_as_float(d.z),
                                      __int_as_float(d.w));
  }
  uint32_t incl = rows;
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  const uint32_t total = __shfl(incl, kWave - 1, 64);
  s_rex[lane] = incl - rows;
  s_cnt[lane] = 0u;
  wave_sync();
  for (uint32_t base = 0; base < total; base += kWave) {
    const uint32_t item = base + static_cast<uint32_t>(lane);
    if (item < total) {
      int own = 0;  // last splat whose first row is <= item
#pragma unroll
      for (int step = 32; step > 0; step >>= 1)
        if (s_rex[own + step] <= item) own += step;
      const float4 u = s_set[3 * own], v = s_set[3 * own + 1], w = s_set[3 * own + 2];
      BandSetup s;
      s.mx = u.x; s.my = u.y; s.A = 0.0f; s.B = u.z; s.det = u.w;
      s.tA = v.x; s.vmax = v.y; s.vr = v.z; s.invA = v.w;
      s.ok = s.det > 0.0f;
      const int4 dd = make_int4(__float_as_int(w.x), __float_as_int(w.y), __float_as_int(w.z), __float_as_int(w.w));
      int tx0;
      const uint32_t nt = row_tiles(s, dd, dd.z / kTile + static_cast<int>(item - s_rex[own]), tx0);
      if (nt) atomicAdd(&s_cnt[own], nt);
    }
  }
  wave_sync();
  return s_cnt[lane];
}

}  // namespace gs
