// Shared device-side definitions for the gfx950 Gaussian-splat kernels.
//
// Numerics policy. Every decision the rasterizer takes (tile membership, alpha >= 1/255,
// early termination) must come out the same on the GPU and in the CPU oracle, so the
// forward path uses only correctly rounded IEEE operations: +, -, *, fma, IEEE division
// and sqrt, rint and ldexp; transcendentals come from gs_math.h. The library is compiled
// with -ffp-contract=off, so every fused multiply-add is an explicit fma().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gs_math.h"

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
constexpr int kListHeader = 4;  // words before the entries of the 3D bucket list ([0] = count)

constexpr float kAlphaMin = 1.0f / 255.0f;
constexpr float kTStop = 1e-4f;
constexpr float kAlphaMax2D = 0.99f;          // 2D rule sets clamp alpha at 0.99
constexpr float kOneMinusAlphaEps = 1e-6f;    // 3D backward floors (1 - alpha)
constexpr float kDilation = 0.3f;             // screen-space low-pass added to cov2d

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

// Orderable 32-bit image of a float: unsigned order equals float order, and -0 and +0 map
// to one key (they compare equal, so a stable sort keeps them in input order).
__device__ __forceinline__ uint32_t float_order_key(float v) {
  const uint32_t u = __float_as_uint(v + 0.0f);
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

// Logical index of workgroup b of n. Workgroups are dealt to the 8 XCDs round-robin
// (b % 8); giving XCD x the contiguous logical range x * (n / 8) ... (a bijection for any n)
// keeps neighbouring radix tiles -- whose runs of one digit are adjacent in the output, often
// in one cache line -- in one L2.
__device__ __forceinline__ int xcd_tile(int b, int n) {
  const int q = n / 8, r = n % 8, x = b % 8, k = b / 8;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + k;
}

}  // namespace gs
