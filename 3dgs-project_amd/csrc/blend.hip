// Alpha blending for all three rule sets (gs_rules.h): the forward (one 16x16 tile per
// 256-lane workgroup), the bucketed backward (one wavefront per 32-entry bucket, each lane
// owning 4 pixels, replaying T from the forward's checkpoints), and the per-pixel backward
// of the 2D surfaces (one thread per pixel, back to front, one atomic per pair).
//
// Pixel layout inside a tile: lane t owns pixel (t % 16, t / 16) in the forward (the
// references' thread-to-pixel map: toy2d/csrc/rasterize.cu:110-113,
// phase0/csrc/macrotile/splat2d_common.h:83-88), so checkpoint [bucket][t] has the
// references' [B, 256, 4] layout. In the backward, lane l of the wavefront owns pixels
// 64 r + l (rows 4 r + l / 16), r = 0..3. 3D only: a splat is evaluated for the 16x4 strip
// of a wavefront only if its pixel bounds overlap the strip's rows; forward, backward and
// oracle apply this rule identically, so the backward replays exactly the forward's splat
// sequence (the purpose of Faster-GS's per-subtile culling, phase1/fastergs_macro.patch:92-104).
#include <limits.h>

#include <type_traits>

#include "gs_host.h"
#include "gs_rules.h"

namespace gs {

// Elongated splats (3D backward). The conic-gradient sums of a splat whose 2D covariance has a
// condition number lambda_max / lambda_min >= kElongKappa are reduced over the wavefront and
// added over the buckets in float64: the preprocess backward's step from the conic to the
// covariance divides by det^2 and amplifies the rounding of float32 sums for such splats by
// about that condition number (a few hundred float32 roundings of partial sums with
// cancellation would move their scale and rotation gradients by 1e-4 of the whole gradient's
// norm). With t = A + C and d = A C - B^2 of the conic (whose condition number is the
// covariance's), lambda_max / lambda_min >= k  <=>  t^2 >= d (1 + k)^2 / k.
constexpr float kElongKappa = 256.0f;
constexpr float kElongC = (1.0f + kElongKappa) * (1.0f + kElongKappa) / kElongKappa;
constexpr uint32_t kElongBit = 1u << 4;  // in a staged splat's strip mask word

__device__ __forceinline__ bool elongated(const float* rp) {
  const float A = rp[2], B = rp[3], C = rp[4];
  const float t = A + C, d = fmaf(A, C, -(B * B));
  return t * t >= kElongC * d;
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

// The strips of ymask (bits s0 ..: strips inside a 3D splat's pixel y-bounds) whose pixels the
// splat's alpha >= 1/255 ellipse can reach, for the tile whose first pixel column is tile_x0.
// With u = row - mean y, the ellipse A v^2 + 2 B u v + C u^2 <= 2 thr (v = column - mean x,
// thr = ln(255 o) from the record) spans columns v in [(-B u - sqrt(q - det u^2)) / A,
// (-B u + sqrt(q - det u^2)) / A], q = 2 thr A, det = A C - B^2, for |u| <= sqrt(q / det). Over a
// strip's pixel-centre rows the right edge is concave in u, largest at u* = -B sqrt(2 thr /
// (C det)) clamped to the strip, the left edge convex, smallest at -u*; a strip is kept when that
// extent reaches the tile's pixel-centre columns. The extent is widened by 0.05 px + 1e-3 of its
// half-width, far above the error of the approximate reciprocals and square roots here and of
// the blends' own float32 evaluation of the boundary (the hardware exp2 included), so a strip is
// dropped only where every pixel has alpha < 1/255: the blends' results do not change. Splats
// with a condition number above about 4096 keep ymask (det then loses too many bits).
// Evaluated for the strips in `want` only (a forward wavefront needs its own strip).
__device__ __forceinline__ uint32_t strip_mask_band(const float* rp, int tile_x0, int tile_y0, uint32_t ymask,
                                                    uint32_t want = 0xfu) {
  ymask &= want;
  const float mx = rp[0], my = rp[1], A = rp[2], B = rp[3], C = rp[4], thr = rp[7];
  const float det = fmaf(A, C, -(B * B));
  const float t = A + C;
  if (ymask == 0u || !(det > 0.0f) || !(A > 0.0f) || !(C > 0.0f) || !(thr > 0.0f) || t * t >= 4096.0f * det)
    return ymask;
  const float q = (thr + thr) * A;
  const float idet = __builtin_amdgcn_rcpf(det);
  const float umax = fmaf(__builtin_amdgcn_sqrtf(q * idet), 1.001f, 0.05f);
  const float us = -B * __builtin_amdgcn_sqrtf((thr + thr) * __builtin_amdgcn_rcpf(C) * idet);
  const float iA = __builtin_amdgcn_rcpf(A);
  const float c0 = (static_cast<float>(tile_x0) + 0.5f) - mx;  // the tile's columns, from the mean
  const float c1 = c0 + static_cast<float>(kTile - 1);
  uint32_t m = 0;
#pragma unroll
  for (int s = 0; s < kStrips; ++s) {
    if (((ymask >> s) & 1u) == 0u) continue;
    const float ya = (static_cast<float>(tile_y0 + kStripRows * s) + 0.5f) - my;
    const float ua = fmaxf(ya, -umax), ub = fminf(ya + static_cast<float>(kStripRows - 1), umax);
    if (ua > ub) continue;
    const float ur = fminf(fmaxf(us, ua), ub), ul = fminf(fmaxf(-us, ua), ub);
    const float sr = __builtin_amdgcn_sqrtf(fmaxf(fmaf(-det * ur, ur, q), 0.0f));
    const float sl = __builtin_amdgcn_sqrtf(fmaxf(fmaf(-det * ul, ul, q), 0.0f));
    const float fr = fmaf(-B, ur, sr) * iA, fl = fmaf(-B, ul, -sl) * iA;
    const float mg = fmaf(1e-3f, fmaxf(fabsf(fr), fabsf(fl)), 0.05f);
    if (fr + mg >= c0 && fl - mg <= c1) m |= 1u << s;
  }
  return m;
}

template <typename S>
struct BlendArgs {
  const S* rec;                    // [n, 16]
  const uint32_t* ranges;          // tile t: [ranges[t * stride], ranges[t * stride + 1])
  int range_stride;                // 2: (T, 2) ranges; 1: (T + 1) CSR offsets
  const uint32_t* point_list;      // [m]
  const uint32_t* bucket_offsets;  // [T + 1] (first bucket of each tile)
  int W, H, tiles_x, n_tiles;
  S bg0, bg1, bg2;
  // forward outputs / backward inputs
  S* image;
  S* final_T;
  S* alpha_out;  // 3D forward (may be null): 1 - final_T
  int32_t* n_contrib;     // 3D, toy2d: last position + 1; phase0: number of splats
  int32_t* last_contrib;  // phase0: last position + 1 (may be null)
  uint32_t* tile_max;     // [T] max over pixels of last position + 1 (may be null in backward)
  S* ckpt;                // [B, 256, 4]
  unsigned long long* counters;  // [3]: atomic adds, checkpoint bytes, splat-pixel evaluations
  // backward
  const uint32_t* bucket_to_tile;
  const uint32_t* n_buckets_dev;  // bucket count on device (may be null)
  int64_t n_buckets;              // grid bound (host)
  const S* grad_image;
  const S* grad_alpha;  // 3D: gradient of alpha = 1 - final_T (may be null)
  S* grad_rec;          // [n, 12]
  // 3D: float64 sums of the conic gradient (A, B, C) of the elongated splats, [n, 4] (may be
  // null: then every splat takes the float32 sums)
  double* conic64;
  // pruning scores (3D): scores[g] += sum over pixels of the blending weight alpha T of g
  float* scores;
  // 3D: buckets the backward reads (appended by the forward, consumed by the backward)
  uint32_t* bucket_list;
  // 3D forward: bucket_to_tile of the tile's buckets (may be null), and a float4 buffer that
  // the workgroups zero between them (may be null; the backward's screen gradients)
  uint32_t* b2t_out;
  float4* clear4;
  int64_t clear4_n;
};

// Per-wavefront counter increment (one atomic per wavefront).
__device__ __forceinline__ void count_add(unsigned long long* c, uint32_t v) {
  uint32_t s = v;
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0 && s) atomicAdd(c, static_cast<unsigned long long>(s));
}

// ---------------------------------------------------------------------------------------
// Wavefront reductions
// ---------------------------------------------------------------------------------------
// Sum over the wavefront, returned to every lane: DPP row shifts reduce each row of 16
// lanes, row_bcast15 / row_bcast31 combine the rows, lane 63 holds the total.
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

// Double: butterfly over lane-crossing shuffles (the 2D surfaces' float64 mode).
__device__ __forceinline__ double wave_sum(double v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Maximum over the wavefront of a non-negative int, every lane active: DPP within the rows of 16
// (quad swaps, half-row and row mirrors), then the rows exchanged with v_permlane16_swap and
// v_permlane32_swap (8 instructions instead of 6 LDS-routed shuffle rounds).
__device__ __forceinline__ int wave_max(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xf, 0xf, false));  // row_mirror
  const auto a = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
  v = max(static_cast<int>(a[0]), static_cast<int>(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
  return max(static_cast<int>(b[0]), static_cast<int>(b[1]));
}

__device__ __forceinline__ float opaque_zero() {
  float z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// Two such zeros from one 64-bit move (in a register pair).
__device__ __forceinline__ void opaque_zero2(float& a, float& b) {
  double z;
  asm volatile("v_mov_b64 %0, 0" : "=v"(z));
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(z));
  a = __uint_as_float(static_cast<uint32_t>(u));
  b = __uint_as_float(static_cast<uint32_t>(u >> 32));
}

// An integer zero in a vector register: an LDS address offset by it is computed once into a
// VGPR, and unrolled reads from it then take their offsets as immediates.
__device__ __forceinline__ int opaque_zero_vgpr() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

__device__ __forceinline__ void atomic_add_grad(float* p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add_grad(double* p, double v) { unsafeAtomicAdd(p, v); }

// ---------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------
// Bucket list written by the 3D forward: [0] buckets the backward reads, [1..3] zero,
// [kListHeader + i] bucket indices (any order).

// Forward blend with a workgroup per tile and a pixel per thread, the tile's list staged 256
// entries at a time for the 4 wavefronts together: the 2D rule sets, float64, the counting
// variant and the pruning scores. (The plain 3D float forward is blend_fwd_strip_kernel.)
// kScore: instead of the image, accumulate every splat's blending weights alpha T over the
// tile's pixels into a.scores (a wavefront sum per splat into LDS, one global atomic per
// staged splat and tile); the blend itself is the forward's, decision for decision.
template <int R, typename S, bool kCount, bool kScore = false>
__global__ __launch_bounds__(kTilePixels) void blend_fwd_kernel(BlendArgs<S> a) {
  using Ru = Rule<R, S>;
  static_assert(!kScore || (R == kRules3D && std::is_same<S, float>::value), "scores: 3D float only");
  __shared__ Staged<S> s_sp[kTilePixels];
  __shared__ uint32_t s_mask[Ru::kStrips ? kTilePixels : 1];
  __shared__ uint32_t s_max;
  __shared__ float s_score[kScore ? kTilePixels : 1];
  __shared__ uint32_t s_gid[kScore ? kTilePixels : 1];

  const int tile = blockIdx.x;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int px = tx * kTile + (t & 15), py = ty * kTile + (t >> 4);
  const bool inside = px < a.W && py < a.H;
  const S pxf = static_cast<S>(px) + Ru::pix_off(), pyf = static_cast<S>(py) + Ru::pix_off();
  const uint32_t r0 = a.ranges[static_cast<int64_t>(tile) * a.range_stride];
  const uint32_t r1 = a.ranges[static_cast<int64_t>(tile) * a.range_stride + 1];
  const int len = static_cast<int>(r1 - r0);
  S* ck = a.ckpt ? a.ckpt + (static_cast<int64_t>(a.bucket_offsets[tile]) * kTilePixels + t) * 4 : nullptr;
  if (t == 0) s_max = 0;
  if (a.b2t_out) {
    // the tile of each of this tile's buckets (what a separate bucket_to_tile pass would write)
    const uint32_t bf = a.bucket_offsets[tile], bl = a.bucket_offsets[tile + 1];
    for (uint32_t b = bf + t; b < bl; b += kTilePixels) a.b2t_out[b] = static_cast<uint32_t>(tile);
  }
  if (a.clear4) {
    // this workgroup's share of the buffer to zero: stores only, hidden under the blend's
    // arithmetic
    const int64_t per = (a.clear4_n + gridDim.x - 1) / gridDim.x;
    const int64_t lo = per * tile, hi = min(lo + per, a.clear4_n);
    for (int64_t q = lo + t; q < hi; q += kTilePixels) a.clear4[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }

  // 3D: a pixel has stopped exactly when T < 1e-4 (T only decreases; pixels outside the
  // image start at T = 0), so no separate per-lane flag is kept
  constexpr bool kStopByT = R == kRules3D;
  S T = (kStopByT && !inside) ? S(0) : S(1), Cr = S(0), Cg = S(0), Cb = S(0);
  int last = 0, count = 0;
  uint32_t evals = 0;
  bool done = !inside;
  int covered = len;  // list positions whose bucket checkpoints the loop wrote
  for (int b0 = 0; b0 < len; b0 += kTilePixels) {
    if (__syncthreads_count((kStopByT ? T < Ru::t_stop() : done) ? 1 : 0) == kTilePixels) {
      covered = b0;
      break;
    }
    const int j = b0 + t;
    if (j < len) {
      const uint32_t g = a.point_list[r0 + j];
      const S* rp = a.rec + static_cast<int64_t>(g) * kRecFloats;
      s_sp[t] = Ru::stage(rp);
      if constexpr (Ru::kStrips)
        s_mask[t] = strip_mask_band(rp, tx * kTile, ty * kTile, strip_mask(reinterpret_cast<const int4*>(rp)[3], ty * kTile));
      if constexpr (kScore) {
        s_gid[t] = g;
        s_score[t] = 0.0f;
      }
    }
    __syncthreads();
    const int nb = min(kTilePixels, len - b0);
    // this wavefront's strip bit of every staged splat, as four 64-bit masks (3D)
    uint64_t wm[4] = {~0ull, ~0ull, ~0ull, ~0ull};
    if constexpr (Ru::kStrips) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int jj = 64 * q + lane;
        wm[q] = __ballot((jj < nb && ((s_mask[jj] >> wave) & 1u)) ? 1 : 0);
      }
    }
    // one 32-entry bucket at a time: its checkpoint, then its splats
    for (int c0 = 0; c0 < nb; c0 += kBucket) {
      if (ck) {
        S* c = ck + static_cast<int64_t>((b0 + c0) / kBucket) * kTilePixels * 4;
        if constexpr (Ru::kCkptTFirst) {
          c[0] = T; c[1] = Cr; c[2] = Cg; c[3] = Cb;
        } else {
          c[0] = Cr; c[1] = Cg; c[2] = Cb; c[3] = T;
        }
      }
      if (__ballot((kStopByT ? T < Ru::t_stop() : done) ? 0 : 1) == 0ull) continue;  // all lanes stopped
      const int c1 = min(c0 + kBucket, nb);
      const uint64_t qm = (c0 < 64) ? wm[0] : (c0 < 128) ? wm[1] : (c0 < 192) ? wm[2] : wm[3];
      uint32_t cm = static_cast<uint32_t>(qm >> (c0 & 63));
      if (c1 - c0 < kBucket) cm &= (1u << (c1 - c0)) - 1u;
      // wave-uniform walk over the splats whose bounds reach this wavefront's rows; the body
      // has no lane branches (a lane that has stopped or rejects the splat composites nothing),
      // so the scalar unit only runs the walk
      auto body = [&](const Staged<S>& sp, int jj) -> bool {
        Eval<S> e;
        const bool live = kStopByT ? T >= Ru::t_stop() : !done;
        if constexpr (kCount) evals += live ? 1u : 0u;
        bool take = Ru::eval(sp, pxf, pyf, e) && live;
        if constexpr (Ru::kStopBefore) {
          const bool stop = take && T * (S(1) - e.alpha) < Ru::t_stop();
          done = done || stop;
          take = take && !stop;
        }
        if constexpr (kScore) {
          if (__ballot(take ? 1 : 0) != 0ull) {
            const float w = wave_sum(take ? e.alpha * T : 0.0f);
            if (lane == 0) atomicAdd(&s_score[jj], w);
          }
        }
        if constexpr (R == kRules3D) {
          // alpha 0 leaves C and T bit-identical (the colours of the records are finite)
          composite<R, S>(Cr, Cg, Cb, T, sp, take ? e.alpha : S(0));
        } else {
          S r = Cr, g = Cg, b = Cb, t = T;
          composite<R, S>(r, g, b, t, sp, e.alpha);
          Cr = take ? r : Cr;
          Cg = take ? g : Cg;
          Cb = take ? b : Cb;
          T = take ? t : T;
        }
        count += take ? 1 : 0;
        if constexpr (!Ru::kStopBefore && !kStopByT) done = done || T < Ru::t_stop();
        return take;
      };
      while (cm != 0u) {
        const int jj = c0 + __builtin_ctz(cm);
        cm &= cm - 1u;
        last = body(s_sp[jj], jj) ? b0 + jj + 1 : last;
      }
    }
    if constexpr (kScore) {
      __syncthreads();  // every wavefront's sums are in
      if (t < nb && s_score[t] != 0.0f) unsafeAtomicAdd(a.scores + s_gid[t], s_score[t]);
    }
  }
  if constexpr (kCount) count_add(a.counters + 2, evals);
  if constexpr (kScore) return;
  if constexpr (R == kRulesPhase0) {
    // phase0 writes every checkpoint slot: buckets after the workgroup stopped keep the
    // final state (phase0/csrc/macrotile/bindings.cpp:167-169)
    if (ck) {
      for (int q = (covered + kBucket - 1) / kBucket; q < (len + kBucket - 1) / kBucket; ++q) {
        S* c = ck + static_cast<int64_t>(q) * kTilePixels * 4;
        c[0] = Cr; c[1] = Cg; c[2] = Cb; c[3] = T;
      }
    }
  } else if constexpr (R == kRulesToy2D) {
    // toy2d leaves the buckets after the workgroup stopped zero (toy2d/csrc/rasterize.cu:131-133,
    // 383, where the state buffer starts zeroed); here they are zeroed by the workgroup itself,
    // so the buffer needs no clearing beforehand
    if (ck) {
      for (int q = (covered + kBucket - 1) / kBucket; q < (len + kBucket - 1) / kBucket; ++q) {
        S* c = ck + static_cast<int64_t>(q) * kTilePixels * 4;
        c[0] = S(0); c[1] = S(0); c[2] = S(0); c[3] = S(0);
      }
    }
  }
  if (inside) {
    const int64_t pix = static_cast<int64_t>(py) * a.W + px;
    if constexpr (Ru::kInterleaved) {
      a.image[3 * pix] = Cr;
      a.image[3 * pix + 1] = Cg;
      a.image[3 * pix + 2] = Cb;
    } else {
      const int64_t HW = static_cast<int64_t>(a.H) * a.W;
      a.image[pix] = fma(T, a.bg0, Cr);
      a.image[HW + pix] = fma(T, a.bg1, Cg);
      a.image[2 * HW + pix] = fma(T, a.bg2, Cb);
    }
    a.final_T[pix] = T;
    if (a.n_contrib) a.n_contrib[pix] = Ru::kCountContrib ? count : last;
    if (a.last_contrib) a.last_contrib[pix] = last;
    if (last > 0) atomicMax(&s_max, static_cast<uint32_t>(last));
  }
  __syncthreads();
  if (t == 0 && a.tile_max) a.tile_max[tile] = s_max;
  if (a.bucket_list) {
    // append the buckets the backward reads: those starting before the tile's last blended entry
    __shared__ uint32_t s_base;
    const uint32_t n_act = (s_max + kBucket - 1) / kBucket;
    if (t == 0) s_base = n_act ? atomicAdd(a.bucket_list, n_act) : 0u;
    __syncthreads();
    const uint32_t first = a.bucket_offsets[tile];
    for (uint32_t k = t; k < n_act; k += kTilePixels) a.bucket_list[kListHeader + s_base + k] = first + k;
  }
}


// 3D forward with the tile's 4 strips split over 4 / P wavefronts. A lane owns the P pixels of
// one column that lie in its wavefront's strips (pixel 64 r + lane of the tile: row 4 r + lane /
// 16, column lane % 16, the pixel layout of the bucketed backward): the column terms of the power
// are computed once per splat for its P pixels, the strip test of pixel r is one scalar bit test,
// and each wavefront stages the tile's list 64 entries at a time in its own LDS, so it waits for
// no other wavefront until the tile's end. Per pixel it takes the decisions of Rule<kRules3D>
// with the operations of the pruning-score pass of blend_fwd_kernel and of the oracle's forward
// (alpha >= 1/255 while T >= 1e-4; composite with alpha 0 otherwise). P = 1 is launched.
template <int P>
__global__ __launch_bounds__(4 * kWave) void blend_fwd_strip_kernel(BlendArgs<float> a) {
  using Ru = Rule<kRules3D, float>;
  constexpr int kWT = kStrips / P;  // wavefronts per tile
  constexpr int kTPB = 4 / kWT;     // tiles per workgroup
  __shared__ Staged<float> s_sp[4][kWave];
  __shared__ uint32_t s_max[kTPB];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = wave % kWT;  // the wavefront's strips: sub P ... sub P + P - 1
  const int tile = static_cast<int>(blockIdx.x) * kTPB + wave / kWT;
  const bool real = tile < a.n_tiles;
  if (lane == 0 && sub == 0) s_max[wave / kWT] = 0u;
  Staged<float>* sw = s_sp[wave];
  const int tt = real ? tile : 0;
  const int tx = tt % a.tiles_x, ty = tt / a.tiles_x;
  const uint32_t r0 = a.ranges[static_cast<int64_t>(tt) * a.range_stride];
  const uint32_t r1 = a.ranges[static_cast<int64_t>(tt) * a.range_stride + 1];
  const int len = real ? static_cast<int>(r1 - r0) : 0;
  const int px = tx * kTile + (lane & 15);
  const float pxf = static_cast<float>(px) + Ru::pix_off();
  float T[P], Cr[P], Cg[P], Cb[P], pyf[P];
  int last[P];
#pragma unroll
  for (int r = 0; r < P; ++r) {
    const int py = ty * kTile + kStripRows * (sub * P + r) + (lane >> 4);
    pyf[r] = static_cast<float>(py) + Ru::pix_off();
    T[r] = (real && px < a.W && py < a.H) ? 1.0f : 0.0f;  // a pixel outside the image has stopped
    Cr[r] = Cg[r] = Cb[r] = 0.0f;
    last[r] = 0;
  }
  const uint32_t bfirst = (real && a.bucket_offsets) ? a.bucket_offsets[tt] : 0u;
  if (real && sub == 0) {
    if (a.b2t_out) {
      const uint32_t bl = a.bucket_offsets[tt + 1];
      for (uint32_t b = bfirst + lane; b < bl; b += kWave) a.b2t_out[b] = static_cast<uint32_t>(tt);
    }
    if (a.clear4) {
      const int64_t per = (a.clear4_n + a.n_tiles - 1) / a.n_tiles;
      const int64_t lo = per * tt, hi = min(lo + per, a.clear4_n);
      for (int64_t q = lo + lane; q < hi; q += kWave) a.clear4[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
  float* ck = a.ckpt ? a.ckpt + (static_cast<int64_t>(bfirst) * kTilePixels + kWave * sub * P + lane) * 4 : nullptr;

  bool stopped = false;
  for (int b0 = 0; b0 < len && !stopped; b0 += kWave) {
    wave_sync();  // every lane is done with the previous batch
    const int j = b0 + lane;
    uint32_t sm = 0;
    if (j < len) {
      const float* rp = a.rec + static_cast<int64_t>(a.point_list[r0 + j]) * kRecFloats;
      sw[lane] = Ru::stage(rp);
      sm = strip_mask_band(rp, tx * kTile, ty * kTile, strip_mask(reinterpret_cast<const int4*>(rp)[3], ty * kTile),
                           ((1u << P) - 1u) << (sub * P)) >> (sub * P);
    }
    // staged entries reaching pixel r of every lane, as 64-bit masks
    uint64_t wm[P];
#pragma unroll
    for (int r = 0; r < P; ++r) wm[r] = __ballot(((sm >> r) & 1u) ? 1 : 0);
    wave_sync();
    const int nb = min(kWave, len - b0);
    for (int c0 = 0; c0 < nb; c0 += kBucket) {
      if (ck) {
        float* c = ck + static_cast<int64_t>((b0 + c0) / kBucket) * kTilePixels * 4;
#pragma unroll
        for (int r = 0; r < P; ++r)
          reinterpret_cast<float4*>(c)[kWave * r] = make_float4(Cr[r], Cg[r], Cb[r], T[r]);
      }
      bool live = false;
#pragma unroll
      for (int r = 0; r < P; ++r) live = live || T[r] >= Ru::t_stop();
      if (__ballot(live ? 1 : 0) == 0ull) {  // every pixel of the wavefront has stopped
        stopped = true;
        break;
      }
      uint32_t cm[P], cany = 0;
#pragma unroll
      for (int r = 0; r < P; ++r) {
        cm[r] = static_cast<uint32_t>(wm[r] >> c0);
        if (nb - c0 < kBucket) cm[r] &= (1u << (nb - c0)) - 1u;
        cm[r] = __builtin_amdgcn_readfirstlane(cm[r]);
        cany |= cm[r];
      }
      const Staged<float>* bp = sw + (c0 + opaque_zero_vgpr());
      int lastk[P];
#pragma unroll
      for (int r = 0; r < P; ++r) lastk[r] = -1;
#pragma unroll
      for (int k = 0; k < kBucket; ++k) {
        if (((cany >> k) & 1u) == 0u) continue;  // wave-uniform
        const Staged<float> sp = bp[k];
        const Ru::Col cl = Ru::col(sp, pxf);
#pragma unroll
        for (int r = 0; r < P; ++r) {
          if (P > 1 && ((cm[r] >> k) & 1u) == 0u) continue;  // wave-uniform strip test
          const float dy = sp.my - pyf[r];
          const float alpha = sp.o * Ru::falloff(Ru::power(sp, cl, dy));
          const bool take = alpha >= Ru::alpha_min() && T[r] >= Ru::t_stop();
          composite<kRules3D, float>(Cr[r], Cg[r], Cb[r], T[r], sp, take ? alpha : 0.0f);
          lastk[r] = take ? k : lastk[r];
        }
      }
#pragma unroll
      for (int r = 0; r < P; ++r) last[r] = lastk[r] >= 0 ? b0 + c0 + lastk[r] + 1 : last[r];
    }
  }

  int lmax = 0;
  const int64_t HW = static_cast<int64_t>(a.H) * a.W;
#pragma unroll
  for (int r = 0; r < P; ++r) {
    const int py = ty * kTile + kStripRows * (sub * P + r) + (lane >> 4);
    if (real && px < a.W && py < a.H) {
      const int64_t pix = static_cast<int64_t>(py) * a.W + px;
      a.image[pix] = fmaf(T[r], a.bg0, Cr[r]);
      a.image[HW + pix] = fmaf(T[r], a.bg1, Cg[r]);
      a.image[2 * HW + pix] = fmaf(T[r], a.bg2, Cb[r]);
      a.final_T[pix] = T[r];
      if (a.alpha_out) a.alpha_out[pix] = 1.0f - T[r];
      if (a.n_contrib) a.n_contrib[pix] = last[r];
      lmax = max(lmax, last[r]);
    }
  }
  lmax = wave_max(lmax);
  if (kWT > 1) {
    __syncthreads();  // s_max cleared
    if (lane == 0 && lmax > 0) atomicMax(&s_max[wave / kWT], static_cast<uint32_t>(lmax));
    __syncthreads();
    lmax = static_cast<int>(s_max[wave / kWT]);
  }
  if (!real || sub != 0) return;
  const uint32_t tmax = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lmax));
  if (lane == 0 && a.tile_max) a.tile_max[tt] = tmax;
  if (a.bucket_list) {
    // append the buckets the backward reads: those starting before the tile's last blended entry
    const uint32_t n_act = (tmax + kBucket - 1) / kBucket;
    uint32_t base = 0;
    if (lane == 0 && n_act) base = atomicAdd(a.bucket_list, n_act);
    base = __shfl(base, 0, 64);
    for (uint32_t k = lane; k < n_act; k += kWave) a.bucket_list[kListHeader + base + k] = bfirst + k;
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Transposing reduction of 12 per-lane values over the wavefront. Each exchange step halves
// the values a lane carries (the partner keeps the other half): xor 32 with
// v_permlane32_swap, xor 16 with v_permlane16_swap, xor 8 with DPP row_ror:8; then the two
// remaining values are summed over their 8-lane group (half-row mirror, quad xor 1, quad xor 2).
// ~30 instructions instead of 12 separate 6-level reductions. On return every lane of group
// g = lane / 8 holds the totals of value indices 6 b5 + 3 b4 + 2 b3 + {0, 1} (b = bits of
// lane; index 3 + 6 b5 + 3 b4 with b3 = 1 does not exist) in u0 and u1.
__device__ __forceinline__ void wave_reduce12(const float* v, float& u0, float& u1) {
  const int lane = threadIdx.x & 63;
  float s[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 6]), false, false);
    s[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float t[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s[i]), __float_as_uint(s[i + 3]), false, false);
    t[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  const bool b3 = (lane & 8) != 0;
  const float send0 = b3 ? t[0] : t[2], keep0 = b3 ? t[2] : t[0];
  const float send1 = b3 ? t[1] : 0.0f, keep1 = b3 ? 0.0f : t[1];
  u0 = keep0 + dpp<0x128>(send0);  // row_ror:8 = partner lane ^ 8
  u1 = keep1 + dpp<0x128>(send1);
  u0 += dpp<0x141>(u0);  // row_half_mirror
  u1 += dpp<0x141>(u1);
  u0 += dpp<0xB1>(u0);  // quad_perm [1,0,3,2]
  u1 += dpp<0xB1>(u1);
  u0 += dpp<0x4E>(u0);  // quad_perm [2,3,0,1]
  u1 += dpp<0x4E>(u1);
}

template <int CTRL>
__device__ __forceinline__ double dpp64(double v) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u & 0xffffffffu), CTRL,
                                                                          0xf, 0xf, false));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), CTRL, 0xf,
                                                                          0xf, false));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

__device__ __forceinline__ uint32_t lo32(double v) {
  return static_cast<uint32_t>(static_cast<uint64_t>(__double_as_longlong(v)) & 0xffffffffu);
}
__device__ __forceinline__ uint32_t hi32(double v) {
  return static_cast<uint32_t>(static_cast<uint64_t>(__double_as_longlong(v)) >> 32);
}
__device__ __forceinline__ double f64_of(uint32_t lo, uint32_t hi) {
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Reduction of one bucket-splat step of the 3D backward without the |dL/dmean2d| sums. In: the
// lane's sums over its 4 pixels (one column) of h, h dy, h dy^2 and the three colour sums, and
// the column's dx. The 4 lanes of a column (lane ^ 16, ^ 32) are summed first, transposing: xor
// 32 with v_permlane32_swap over the pairs (h, red), (h dy, green), (h dy^2, blue), leaving the
// h sums in lanes 0-31 and the colour sums in lanes 32-63; xor 16 with v_permlane16_swap, the
// first sum in all 4 rows of 16 lanes and the other two split between even and odd rows. Only
// then are the dx factors applied, once per column instead of once per lane, in row 0 alone
// (f = dx there, 1 elsewhere). The four values of every lane are then summed over the 16 columns
// of its row: xor 8 with DPP row_ror:8 over the pairs, then the 8-lane group sums (half-row
// mirror, quad xor 1, quad xor 2). On return group g = lane / 8 holds in (u0, u1):
//   g 0: (sum h dx, sum h dy)          g 1: (sum h dx^2, sum h dx dy)
//   g 2: (sum h, sum h dy^2)           g 4: (red, green)       g 6: (red, blue)
// (g 3, 5, 7 hold repeats). 27 instructions, the dx products included.
__device__ __forceinline__ void wave_reduce_cols(float sh, float shy, float shyy, float cr, float cg, float cb,
                                                 float dx, bool row0, float& u0, float& u1) {
  const int lane = threadIdx.x & 63;
  float s0, s1, s2;
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sh), __float_as_uint(cr), false, false);
    s0 = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(shy), __float_as_uint(cg), false, false);
    s1 = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(shyy), __float_as_uint(cb), false, false);
    s2 = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float t0, t1;
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s0), __float_as_uint(s0), false, false);
    t0 = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // every row: its quarter's first sum
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s1), __float_as_uint(s2), false, false);
    t1 = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // even rows s1, odd rows s2
  }
  const float f = row0 ? dx : 1.0f;
  const float v0 = t0 * f, v1 = v0 * f, v3 = t1 * f;
  const bool b3 = (lane & 8) != 0;
  u0 = (b3 ? v1 : v0) + dpp<0x128>(b3 ? v0 : v1);  // row_ror:8 = partner lane ^ 8
  u1 = (b3 ? v3 : t1) + dpp<0x128>(b3 ? t1 : v3);
  u0 += dpp<0x141>(u0);  // row_half_mirror
  u1 += dpp<0x141>(u1);
  u0 += dpp<0xB1>(u0);  // quad_perm [1,0,3,2]
  u1 += dpp<0xB1>(u1);
  u0 += dpp<0x4E>(u0);  // quad_perm [2,3,0,1]
  u1 += dpp<0x4E>(u1);
  // (the totals are formed here, with every lane active, so that the DPP moves fold into the
  // adds rather than the adds sinking into the owners' branch)
  asm volatile("" : "+v"(u0), "+v"(u1));
}

__device__ __forceinline__ void wave_reduce12(const double* v, double& u0, double& u1) {
  // float64 (2D surfaces): full butterflies, then the float path's placement of the totals
  const int g = (threadIdx.x & 63) >> 3;
  const int base = 6 * (g >> 2) + 3 * ((g >> 1) & 1) + 2 * (g & 1);
  u0 = 0.0;
  u1 = 0.0;
#pragma unroll
  for (int k = 0; k < 12; ++k) {
    const double t = wave_sum(v[k]);
    if (k == base) u0 = t;
    if (k == base + 1) u1 = t;
  }
}

// Raw per-pair sums of the bucketed backward (the splat-constant factors are applied once
// per splat in finish_grad): [0] sum h dx (phase0: h a), [1] sum h dy (phase0: h b),
// [2] sum h dx dx (h a dx), [3] sum h dx dy (h a dy), [4] sum h dy dy (h b dy), [5] sum G dL/dalpha,
// [6..8] colour, [9..10] |dL/dmean| (3D); h = alpha dL/dalpha = dL/dpower.
template <int R, typename S>
__device__ __forceinline__ void pair_sums(const Staged<S>& s, const Eval<S>& e, S dLda, S* acc) {
  if (e.clamped) return;
  acc[5] = fma(e.G, dLda, acc[5]);
  const S h = e.alpha * dLda;
  S hx, hy;
  if constexpr (R == kRulesPhase0) {
    hx = h * e.a;
    hy = h * e.b;
    acc[2] = fma(hx, e.dx, acc[2]);
    acc[3] = fma(hx, e.dy, acc[3]);
    acc[4] = fma(hy, e.dy, acc[4]);
  } else {
    hx = h * e.dx;
    hy = h * e.dy;
    acc[2] = fma(hx, e.dx, acc[2]);
    acc[3] = fma(hx, e.dy, acc[3]);
    acc[4] = fma(hy, e.dy, acc[4]);
    if constexpr (R == kRules3D) {
      acc[9] += fabs(fma(s.n0, hx, s.n1 * hy));
      acc[10] += fabs(fma(s.n1, hx, s.nat2 * hy));
    }
  }
  acc[0] += hx;
  acc[1] += hy;
}

// Final gradient of value index k from its total u (u0, u1: totals of indices 0 and 1).
template <int R, typename S>
__device__ __forceinline__ S finish_grad(const Staged<S>& s, int k, S u, S u0, S u1) {
  if constexpr (R == kRulesPhase0) {
    // power = -(a^2 + b^2) / 2 with a = l0 dx + l1 dy, b = l2 dy, d = pixel - mean
    if (k == 0) return s.s0 * u0;
    if (k == 1) return fma(s.s1, u0, s.s2 * u1);
    if (k >= 2 && k <= 4) return -u;
    if (k == 5) return u * s.o * (S(1) - s.o);  // dL/dlogit = dL/do o (1 - o)
    return u;
  } else {
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
    // power = -1/2 (A dx^2 + 2 B dx dy + C dy^2), d = mean - pixel
    if (k == 0) return -fma(A, u0, B * u1);
    if (k == 1) return -fma(B, u0, C * u1);
    if (k == 2 || k == 4) return S(-0.5) * u;
    if (k == 3) return -u;
    return u;
  }
}

// ---------------------------------------------------------------------------------------
// Bucketed backward
// ---------------------------------------------------------------------------------------
// Wavefronts per workgroup of the bucketed backward. Each wavefront takes its own bucket and
// shares nothing with the others, so a workgroup of one lets a CU take the next bucket as soon
// as any wavefront ends: 3D (1M SH3: 199.3 -> 195.7 us against four per workgroup) and phase0
// (0.255 -> 0.242 ms at 50k splats); the toy2d surface keeps four (512^2, 50k: 0.087 against
// 0.098 ms with one).
constexpr int kXcdRun = 4;  // consecutive bucket-list entries per XCD (one-wavefront workgroups)
template <int R>
constexpr int bwd_waves() {
  return R == kRulesToy2D ? 4 : 1;
}
// Staged entries that hold the 3D backward's coefficient table (65 floats)
constexpr int kCoefSlots = ((kWave + 1) * 4 + static_cast<int>(sizeof(Staged<float>)) - 1) /
                           static_cast<int>(sizeof(Staged<float>));
static_assert(sizeof(Staged<float>) == 48 && offsetof(Staged<float>, n0) == 36 && offsetof(Staged<float>, n1) == 40 &&
                  offsetof(Staged<float>, nat2) == 44,
              "the 3D backward reads (n0, n1) and (n1, nat2) as float pairs of a staged splat");

// kAbs (3D): also accumulate |dL/dmean2d| (grad2d slots 9-10) for densification by absolute
// gradient, as Faster-GS's compute_abs_grad instantiation does; without it those slots are
// left untouched.
// One bucket b, by one wavefront (whose LDS slots are s_sp, s_m, s_id).
template <int R, typename S, bool kCount, bool kAbs>
__device__ __forceinline__ void bwd_bucket(const BlendArgs<S>& a, int64_t b, Staged<S>* s_sp, uint32_t* s_m,
                                           uint32_t* s_id, float* s_c, uint32_t& evals, uint32_t& atomics) {
  using Ru = Rule<R, S>;
  constexpr int NV = Ru::kGradVals;
  // (opaque: in the striding kernel the lane's constants are then formed per bucket instead of
  // being hoisted out of its loop and held in registers across it)
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));
  const uint32_t tile = a.bucket_to_tile[b];
  const int bstart = static_cast<int>(b - a.bucket_offsets[tile]) * kBucket;
  const int tmax = a.tile_max ? static_cast<int>(a.tile_max[tile]) : INT_MAX;
  if (bstart >= tmax) return;
  const uint32_t r0 = a.ranges[static_cast<int64_t>(tile) * a.range_stride];
  const uint32_t r1 = a.ranges[static_cast<int64_t>(tile) * a.range_stride + 1];
  const int bsize = min(kBucket, min(static_cast<int>(r1 - r0), tmax) - bstart);
  if (bsize <= 0) return;
  const int tx = static_cast<int>(tile) % a.tiles_x, ty = static_cast<int>(tile) / a.tiles_x;

  uint32_t mk_lane = 0;  // the strip mask of this lane's staged splat (3D)
  if (lane < bsize) {
    const uint32_t g = a.point_list[r0 + bstart + lane];
    const S* rp = a.rec + static_cast<int64_t>(g) * kRecFloats;
    s_sp[lane] = Ru::stage(rp);
    if constexpr (Ru::kStrips) {
      uint32_t mk = strip_mask(reinterpret_cast<const int4*>(rp)[3], ty * kTile);
      if constexpr (R == kRules3D) {
        mk = strip_mask_band(rp, tx * kTile, ty * kTile, mk);
        if (a.conic64 && elongated(rp)) mk |= kElongBit;
        mk_lane = mk;
      } else {
        s_m[lane] = mk;
      }
    }
    s_id[lane] = g;
  }

  // per-pixel state: pixel p = 64 r + lane, row 4 r + lane / 16, column lane % 16
  const int64_t HW = static_cast<int64_t>(a.H) * a.W;
  const int px = tx * kTile + (lane & 15);
  const S pxf = static_cast<S>(px) + Ru::pix_off();
  S T[kPixPerLane], rho[kPixPerLane], Gr[kPixPerLane], Gg[kPixPerLane], Gb[kPixPerLane];
  S pyf[kPixPerLane];
  int lim[kPixPerLane];
  int lim_max = 0;
#pragma unroll
  for (int r = 0; r < kPixPerLane; ++r) {
    const int py = ty * kTile + kStripRows * r + (lane >> 4);
    pyf[r] = static_cast<S>(py) + Ru::pix_off();
    T[r] = S(0);
    rho[r] = S(0);
    Gr[r] = Gg[r] = Gb[r] = S(0);
    lim[r] = 0;
    if (px < a.W && py < a.H) {
      const int64_t pix = static_cast<int64_t>(py) * a.W + px;
      // phase0 without a limit table: every inside pixel replays the bucket and stops by the
      // T < 1e-4 rule (phase0/csrc/macrotile/splat2d_bwd_splat.cu:69)
      const int32_t* lp = a.last_contrib ? a.last_contrib : a.n_contrib;
      const int used = lp ? lp[pix] - bstart : kBucket;
      if (used > 0) {
        lim[r] = used;
        lim_max = max(lim_max, used);
        S img0, img1, img2;
        if constexpr (Ru::kInterleaved) {
          Gr[r] = a.grad_image[3 * pix];
          Gg[r] = a.grad_image[3 * pix + 1];
          Gb[r] = a.grad_image[3 * pix + 2];
          img0 = a.image[3 * pix];
          img1 = a.image[3 * pix + 1];
          img2 = a.image[3 * pix + 2];
        } else {
          Gr[r] = a.grad_image[pix];
          Gg[r] = a.grad_image[HW + pix];
          Gb[r] = a.grad_image[2 * HW + pix];
          img0 = a.image[pix];
          img1 = a.image[HW + pix];
          img2 = a.image[2 * HW + pix];
        }
        const S* c = a.ckpt + (b * kTilePixels + kWave * r + lane) * 4;
        S c0, c1, c2;
        if constexpr (Ru::kCkptTFirst) {
          T[r] = c[0]; c0 = c[1]; c1 = c[2]; c2 = c[3];
        } else {
          c0 = c[0]; c1 = c[1]; c2 = c[2]; T[r] = c[3];
        }
        // rho = G . (image - C): the colour still to come (background included)
        rho[r] = Gr[r] * (img0 - c0) + Gg[r] * (img1 - c1) + Gb[r] * (img2 - c2);
        // alpha = 1 - T_final output: its gradient enters like a background term
        if constexpr (R == kRules3D) {
          if (a.grad_alpha) rho[r] -= a.grad_alpha[pix] * a.final_T[pix];
        }
      }
    }
  }
  if constexpr (R == kRules3D && !kAbs) {
    // the coefficient pair of each lane's gradient, g = -(c0 u0 + c1 u1) of the reduction's totals
    // (u0, u1); lanes 0 and 1 read theirs, the splat's (A, B) and (B, C), from the staged splat,
    // lane l >= 2 reads (t[l], t[l + 1]) of this table (consecutive words: no bank conflicts): the
    // owners' pairs are lane 8 (1/2, 0), 9 (0, 1), 16 (-1, 0), 17 (0, 1/2), 32 (-1, 0), 33 (0, -1),
    // 49 (0, -1), all others (0, 0)
    float* kt = reinterpret_cast<float*>(s_sp + kBucket);
    kt[lane] = lane == 8 || lane == 18 ? 0.5f
               : lane == 10            ? 1.0f
               : (lane == 16 || lane == 32 || lane == 34 || lane == 50) ? -1.0f
                                                                       : 0.0f;
    if (lane == 0) kt[kWave] = 0.0f;
  }
  // (scalar: the splat loop is uniform over the wavefront)
  const int jmax = __builtin_amdgcn_readfirstlane(min(bsize, wave_max(lim_max)));
  wave_sync();

  // value index k owned by this lane after wave_reduce12 (lo = 0 or 1 within the 8-lane group)
  const int grp = lane >> 3, lo = lane & 7;
  const int kidx = 6 * (grp >> 2) + 3 * ((grp >> 1) & 1) + 2 * (grp & 1) + lo;
  const bool owner = lo < 2 && (2 * (grp & 1) + lo) < 3 && kidx < NV;
  if constexpr (R == kRules3D) {
    // The lane's 4 pixels share a column: the column terms of the power and of the mean
    // gradient are computed once per splat, and per pixel only dy-dependent sums are kept;
    // the dx factors are applied in the reduction, once per column. Pixel r of every
    // lane lies in strip r, so the strip test and the wavefront's largest limit of row r are
    // scalar; inside, the pixel body has no branches: a lane past its limit or below the
    // alpha threshold blends alpha = 0, which leaves its T, rho and every sum unchanged.
    // dL/dopacity = sum G dL/dalpha = (sum alpha dL/dalpha) / o: the sum h is reduced instead.
    int lim_row[kPixPerLane];
#pragma unroll
    for (int r = 0; r < kPixPerLane; ++r) lim_row[r] = __builtin_amdgcn_readfirstlane(wave_max(lim[r]));
    // the staged splats' strip bits and elongation bit as scalar bit planes (bit j: splat j), so
    // the per-splat tests below are scalar bit tests with no LDS read
    uint64_t plane[kPixPerLane + 1];
#pragma unroll
    for (int r = 0; r < kPixPerLane; ++r) plane[r] = __ballot(((mk_lane >> r) & 1u) ? 1 : 0);
    plane[kPixPerLane] = __ballot((mk_lane & kElongBit) ? 1 : 0);
    // With |dL/dmean2d| (kAbs) the 12 sums are reduced by wave_reduce12 and the final gradient of
    // the lane's value index k is c0 u0 + c1 u1 + c u (u = its own total): k 0, 1 (mean2d):
    // -(A u0 + B u1), -(B u0 + C u1); k 2, 4: -u/2; k 3: -u; k 5 (opacity): u; colour and
    // |dL/dmean2d|: u. Without, wave_reduce_cols leaves two totals (u0, u1) in each 8-lane group
    // and the gradient of a lane is -(c0 u0 + c1 u1): lanes 0 and 1 the mean2d values from
    // (sum h dx, sum h dy), with (c0, c1) = (A, B) and (B, C) read from the staged splat; lanes 8
    // and 9 the conic A and B (-u0/2, -u1), lanes 16 and 17 the opacity (u0) and the conic C
    // (-u1/2), lanes 32, 33 and 49 the colour, their pairs read from a table of constants.
    // The opacity column holds sum h = sum alpha dL/dalpha = opacity dL/dopacity: the preprocess
    // backward divides by the opacity once per Gaussian (in float64) instead of every
    // bucket-splat step here. The lane-constant parts are chosen here.
    const bool k0 = kidx == 0, k1 = kidx == 1;  // (kAbs) the lanes of the two mean2d values
    int kslot;  // the grad2d column of the lane's gradient (-1: none)
    float kc = 0.0f;
    if constexpr (kAbs) {
      kslot = owner ? kidx : -1;
      kc = (kslot == 2 || kslot == 4) ? -0.5f : kslot == 3 ? -1.0f : kslot >= 5 ? 1.0f : 0.0f;
    } else {
      kslot = lane == 0    ? 0
              : lane == 1  ? 1
              : lane == 8  ? 2
              : lane == 9  ? 3
              : lane == 16 ? 5
              : lane == 17 ? 4
              : lane == 32 ? 6
              : lane == 33 ? 7
              : lane == 49 ? 8
                           : -1;
    }
    // (without kAbs) the float index of the lane's coefficient pair in s_sp, j * m01 + cidx:
    // lanes 0 and 1 in staged splat j, the others in the table after the staged splats
    constexpr int kStagedFloats = static_cast<int>(sizeof(Staged<S>) / sizeof(S));
    const int m01 = lane < 2 ? kStagedFloats : 0;
    const int cidx = lane < 2 ? static_cast<int>(offsetof(Staged<S>, n0) / sizeof(S)) + lane
                              : kBucket * kStagedFloats + lane;
    const bool row0 = lane < 16;
    const bool live_owner = kslot >= 0;
    const bool conic_owner = kslot >= 2 && kslot <= 4;
    const int64_t kofs = kslot;
    for (int j = 0; j < jmax; ++j) {
      const Staged<S> sp = s_sp[j];
      const typename Ru::Col cl = Ru::col(sp, pxf);
      const float n0dx = sp.n0 * cl.dx, n1dx = sp.n1 * cl.dx;
      // zeros the compiler cannot see through: each sum then lives in one register from its
      // zero to its last update, instead of being re-zeroed on every path that skips a pixel
      float sh, shy, shyy, cr, cg, cb;
      opaque_zero2(sh, shy);
      opaque_zero2(shyy, cr);
      opaque_zero2(cg, cb);
      float ab0 = 0.0f, ab1 = 0.0f;
      if constexpr (kAbs) {
        ab0 = opaque_zero();
        ab1 = opaque_zero();
      }
      uint64_t used = 0;  // the lanes that blended the splat (a lane mask: scalar)
#pragma unroll
      for (int r = 0; r < kPixPerLane; ++r) {
        if (((plane[r] >> j) & 1u) == 0u || j >= lim_row[r]) continue;  // wave-uniform
        const bool live = j < lim[r];
        if constexpr (kCount) evals += live ? 1u : 0u;
        const float dy = sp.my - pyf[r];
        const float G = Ru::falloff(Ru::power(sp, cl, dy));
        const float a_raw = sp.o * G;
        const bool above = a_raw >= kAlphaMin;
        const bool take = live && above;
        // (the masks of the two compares themselves: a ballot of their conjunction would first
        // turn it into a per-lane value)
        used |= __builtin_amdgcn_ballot_w64(live) & __builtin_amdgcn_ballot_w64(above);
        const float alpha = take ? a_raw : 0.0f;
        const float w = T[r] * alpha;
        const float dot = fmaf(Gb[r], sp.cb, fmaf(Gg[r], sp.cg, Gr[r] * sp.cr));
        cr = fmaf(w, Gr[r], cr);
        cg = fmaf(w, Gg[r], cg);
        cb = fmaf(w, Gb[r], cb);
        rho[r] = fmaf(-w, dot, rho[r]);
        const float oma = 1.0f - alpha;
        const float dLda = fmaf(T[r], dot, -(rho[r] * __builtin_amdgcn_rcpf(fmaxf(oma, kOneMinusAlphaEps))));
        const float h = alpha * dLda;  // dL/dpower
        const float hy = h * dy;
        sh += h;
        shy += hy;
        shyy = fmaf(hy, dy, shyy);
        if constexpr (kAbs) {
          ab0 = fmaf(fabsf(h), fabsf(fmaf(sp.n1, dy, n0dx)), ab0);
          ab1 = fmaf(fabsf(h), fabsf(fmaf(sp.nat2, dy, n1dx)), ab1);
        }
        T[r] = T[r] * oma;
      }
      if (used == 0) continue;
      const bool wide = ((plane[kPixPerLane] >> j) & 1u) != 0u;  // wave-uniform
      if (wide) {
        // each lane parks the conic sums of its pixels, read back after the float32 reduction
        const float dxsh = cl.dx * sh;
        s_c[lane] = cl.dx * dxsh;
        s_c[kWave + lane] = cl.dx * shy;
        s_c[2 * kWave + lane] = shyy;
      }
      float g;
      if constexpr (kAbs) {
        const float dxsh = cl.dx * sh;
        const float cxx = cl.dx * dxsh, cxy = cl.dx * shy;  // the conic sums of the lane's column
        const float c0 = k0 ? -sp.n0 : k1 ? -sp.n1 : 0.0f;
        const float c1 = k0 ? -sp.n1 : k1 ? -sp.nat2 : 0.0f;
        S acc[12] = {dxsh, shy, cxx, cxy, shyy, sh, cr, cg, cb, ab0, ab1, 0.0f};
        S u0, u1;
        wave_reduce12(acc, u0, u1);
        g = fmaf(c0, u0, fmaf(c1, u1, kc * (lo == 0 ? u0 : u1)));
      } else {
        float u0, u1;
        wave_reduce_cols(sh, shy, shyy, cr, cg, cb, cl.dx, row0, u0, u1);
        const S* cp = reinterpret_cast<const S*>(s_sp) + (j * m01 + cidx);
        g = fmaf(-cp[0], u0, -(cp[1] * u1));
      }
      // (an elongated splat's conic sums go to the float64 buffer below instead)
      if (live_owner && !(wide && conic_owner))
        atomic_add_grad(a.grad_rec + static_cast<int64_t>(s_id[j]) * kGrad2D + kofs, g);
      if (wide) {  // the conic sums in float64
        const uint32_t id = __builtin_amdgcn_readfirstlane(s_id[j]);  // wave-uniform
        wave_sync();  // every lane's parked values
        // row k of 16 lanes (k < 3) sums value k of the 64 lanes: 4 values per lane in float64
        // (exactly), then the row's 16 partial sums; A, B, C = -1/2, -1, -1/2 times the sums of
        // dx^2 h, dx dy h, dy^2 h
        int ln = lane;
        asm volatile("" : "+v"(ln));  // formed here, not kept in registers over the whole loop
        const int k = ln >> 4, r16 = ln & 15;
        double t = 0.0;
        if (k < 3) {
          const float* v = s_c + k * kWave + r16;
          t = (static_cast<double>(v[0]) + static_cast<double>(v[16])) +
              (static_cast<double>(v[32]) + static_cast<double>(v[48]));
        }
        t += dpp64<0x128>(t);  // row_ror:8
        t += dpp64<0x141>(t);  // row_half_mirror
        t += dpp64<0xB1>(t);   // quad_perm [1,0,3,2]
        t += dpp64<0x4E>(t);   // quad_perm [2,3,0,1]
        if (r16 == 0 && k < 3) atomic_add_grad(a.conic64 + 4 * static_cast<uint64_t>(id) + k, (k == 1 ? -1.0 : -0.5) * t);
        // marks the splat's row for the preprocess backward, which then adds the float64 sums
        if (lane == 48) a.grad_rec[static_cast<uint64_t>(id) * kGrad2D + 11] = 1.0f;
        wave_sync();  // the parked values are read before the next splat parks its own
      }
      if constexpr (kCount) atomics += kAbs ? NV : 9;
    }
  } else
  for (int j = 0; j < jmax; ++j) {
    const Staged<S> sp = s_sp[j];
    uint32_t m = 0xfu;
    if constexpr (Ru::kStrips) m = s_m[j];
    S acc[12];
#pragma unroll
    for (int k = 0; k < 12; ++k) acc[k] = S(0);
    bool used = false;
#pragma unroll
    for (int r = 0; r < kPixPerLane; ++r) {
      if (((m >> r) & 1u) == 0u) continue;  // wave-uniform
      if (j >= lim[r]) continue;
      if constexpr (R == kRulesPhase0) {
        if (T[r] < Ru::t_stop()) continue;
      }
      Eval<S> e;
      if constexpr (kCount) ++evals;
      if (!Ru::eval(sp, pxf, pyf[r], e)) continue;
      used = true;
      const S w = T[r] * e.alpha;
      const S dot = fma(Gb[r], sp.cb, fma(Gg[r], sp.cg, Gr[r] * sp.cr));
      acc[6] = fma(w, Gr[r], acc[6]);
      acc[7] = fma(w, Gg[r], acc[7]);
      acc[8] = fma(w, Gb[r], acc[8]);
      rho[r] = fma(-w, dot, rho[r]);
      const S oma = S(1) - e.alpha;
      S dLda;
      if constexpr (R == kRules3D) {
        dLda = fma(T[r], dot, -(rho[r] * __builtin_amdgcn_rcpf(fmaxf(oma, kOneMinusAlphaEps))));
      } else {
        dLda = T[r] * dot - rho[r] / oma;
      }
      pair_sums<R, S>(sp, e, dLda, acc);
      T[r] = T[r] * oma;
    }
    if (__ballot(used ? 1 : 0) == 0) continue;  // wave-uniform
    S u0, u1;
    wave_reduce12(acc, u0, u1);
    if (owner) {
      const S u = lo == 0 ? u0 : u1;
      atomic_add_grad(a.grad_rec + static_cast<int64_t>(s_id[j]) * kGrad2D + kidx,
                      finish_grad<R, S>(sp, kidx, u, u0, u1));
    }
    if constexpr (kCount) atomics += NV;
  }
}

// kList 0: wavefront i takes bucket i of the table. With a.bucket_list (3D), the forward's list
// of the buckets with blended entries: kList 1, wavefront i takes entry i (a wavefront past the
// list's length only reads that length); kList 2, a bounded grid strides over the list (the
// loop keeps more registers live, so it is used only when the table is much longer).
template <int R, typename S, bool kCount, bool kAbs = true, int kList = 0>
__global__ __launch_bounds__(bwd_waves<R>() * kWave) void blend_bwd_bucket_kernel(
    BlendArgs<S> a) {
  constexpr int kBwdWaves = bwd_waves<R>();
  // (3D: the lanes' coefficient table after the wavefront's staged splats)
  __shared__ Staged<S> s_sp[kBwdWaves][kBucket + (R == kRules3D ? kCoefSlots : 0)];
  __shared__ uint32_t s_m[kBwdWaves][kBucket];
  __shared__ uint32_t s_id[kBwdWaves][kBucket];
  // 3D: an elongated splat's three per-lane conic sums, parked over the float32 reduction
  __shared__ float s_c[R == kRules3D ? kBwdWaves : 1][3 * kWave];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float* s_cw = s_c[R == kRules3D ? wave : 0];
  uint32_t evals = 0, atomics = 0;
  if constexpr (kList == 1) {
    // one wavefront per list entry; wavefronts past the list's length leave at once. (One
    // wavefront per workgroup: workgroup b runs on XCD b % 8, and the k-th workgroup of an XCD
    // takes entry (k / kXcdRun * 8 + b % 8) * kXcdRun + k % kXcdRun, so that runs of kXcdRun
    // consecutive entries -- a tile's buckets, which read the same pixels -- share an L2.)
    int64_t i = static_cast<int64_t>(blockIdx.x) * kBwdWaves + wave;
    if constexpr (kBwdWaves == 1) {
      const int64_t k = blockIdx.x / 8;
      i = (k / kXcdRun * 8 + blockIdx.x % 8) * kXcdRun + k % kXcdRun;
    }
    if (i < static_cast<int64_t>(a.bucket_list[0]))
      bwd_bucket<R, S, kCount, kAbs>(a, a.bucket_list[kListHeader + i], s_sp[wave], s_m[wave], s_id[wave], s_cw, evals,
                                     atomics);
  } else if constexpr (kList == 2) {
    // a bounded grid strides over the list (for bucket tables far longer than the list)
    const int64_t cnt = a.bucket_list[0];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBwdWaves;
    // the wavefront's index made scalar: the loop state and the LDS slots' addresses then live in
    // scalar registers (64 VGPRs and 105 SGPRs, 7 wavefronts per SIMD by the SGPRs, against 77
    // VGPRs and 6)
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    float* s_cws = s_c[R == kRules3D ? wave_s : 0];
    if constexpr (kBwdWaves == 1) {
      // logical entries L = blockIdx.x + t * gridDim.x (gridDim.x a multiple of 8 kXcdRun) taken
      // through the list walk's XCD runs (a bijection on every aligned group of 8 kXcdRun), so
      // that a tile's consecutive buckets share an L2 here too
      const int64_t cnt_r = (cnt + 8 * kXcdRun - 1) / (8 * kXcdRun) * (8 * kXcdRun);
      for (int64_t L = blockIdx.x; L < cnt_r; L += stride) {
        const int64_t k = L / 8;
        const int64_t i = (k / kXcdRun * 8 + L % 8) * kXcdRun + k % kXcdRun;
        if (i < cnt)
          bwd_bucket<R, S, kCount, kAbs>(a, a.bucket_list[kListHeader + i], s_sp[wave_s], s_m[wave_s], s_id[wave_s],
                                         s_cws, evals, atomics);
      }
    } else {
      for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBwdWaves + wave_s; i < cnt; i += stride)
        bwd_bucket<R, S, kCount, kAbs>(a, a.bucket_list[kListHeader + i], s_sp[wave_s], s_m[wave_s], s_id[wave_s],
                                       s_cws, evals, atomics);
    }
  } else {
    int64_t b = static_cast<int64_t>(blockIdx.x) * kBwdWaves + wave;
    if constexpr (kBwdWaves == 1) {  // the table walk takes the same XCD runs as the list walk
      const int64_t k = blockIdx.x / 8;
      b = (k / kXcdRun * 8 + blockIdx.x % 8) * kXcdRun + k % kXcdRun;
    }
    if (b < a.n_buckets && !(a.n_buckets_dev && b >= static_cast<int64_t>(*a.n_buckets_dev)))
      bwd_bucket<R, S, kCount, kAbs>(a, b, s_sp[wave], s_m[wave], s_id[wave], s_cw, evals, atomics);
  }
  if constexpr (kCount) {
    if (lane == 0 && atomics) atomicAdd(a.counters, static_cast<unsigned long long>(atomics));
    count_add(a.counters + 2, evals);
  }
}

// ---------------------------------------------------------------------------------------
// Per-pixel backward (2D surfaces): each thread walks its pixel's list back to front,
// recovers T by dividing by (1 - alpha), and issues one atomic per parameter per pair
// (toy2d/csrc/rasterize.cu:182-258, phase0/csrc/macrotile/splat2d_bwd_pixel.cu:13-62).
// ---------------------------------------------------------------------------------------
template <int R, typename S>
__global__ __launch_bounds__(kTilePixels) void blend_bwd_pixel_kernel(BlendArgs<S> a) {
  using Ru = Rule<R, S>;
  __shared__ Staged<S> s_sp[kTilePixels];
  __shared__ uint32_t s_id[kTilePixels];

  const int tile = blockIdx.x;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int t = threadIdx.x;
  const int px = tx * kTile + (t & 15), py = ty * kTile + (t >> 4);
  const bool inside = px < a.W && py < a.H;
  const S pxf = static_cast<S>(px) + Ru::pix_off(), pyf = static_cast<S>(py) + Ru::pix_off();
  const uint32_t r0 = a.ranges[static_cast<int64_t>(tile) * a.range_stride];
  const uint32_t r1 = a.ranges[static_cast<int64_t>(tile) * a.range_stride + 1];
  const int len = static_cast<int>(r1 - r0);
  const int64_t pix = static_cast<int64_t>(py) * a.W + px;
  const int64_t HW = static_cast<int64_t>(a.H) * a.W;

  S Tcur = S(0), G0 = S(0), G1 = S(0), G2 = S(0), bg_dot = S(0), T_final = S(0);
  int lim = 0;
  if (inside) {
    T_final = a.final_T[pix];
    Tcur = T_final;
    lim = (a.last_contrib ? a.last_contrib : a.n_contrib)[pix];
    if constexpr (Ru::kInterleaved) {
      G0 = a.grad_image[3 * pix];
      G1 = a.grad_image[3 * pix + 1];
      G2 = a.grad_image[3 * pix + 2];
    } else {
      G0 = a.grad_image[pix];
      G1 = a.grad_image[HW + pix];
      G2 = a.grad_image[2 * HW + pix];
    }
    if constexpr (Ru::kBackground) bg_dot = a.bg0 * G0 + a.bg1 * G1 + a.bg2 * G2;
  }
  S acc0 = S(0), acc1 = S(0), acc2 = S(0);  // colour behind the current splat, over T
  uint32_t evals = 0, atomics = 0;
  // toy2d: the wavefront's contributions to a splat reduced before the atomics (the phase0
  // surface keeps one atomic per pixel and value: its backward A is that method, counted)
  constexpr bool kPreReduce = R == kRulesToy2D;
  const int lane = t & 63;
  const int grp = lane >> 3, lo = lane & 7;
  const int kidx = 6 * (grp >> 2) + 3 * ((grp >> 1) & 1) + 2 * (grp & 1) + lo;
  const bool owner = lo < 2 && (2 * (grp & 1) + lo) < 3 && kidx < 9;
  for (int b0 = 0; b0 < len; b0 += kTilePixels) {
    __syncthreads();  // the previous batch is no longer in use
    const int k = len - 1 - (b0 + t);  // position in the tile list, back to front
    if (k >= 0) {
      const uint32_t g = a.point_list[r0 + k];
      s_sp[t] = Ru::stage(a.rec + static_cast<int64_t>(g) * kRecFloats);
      s_id[t] = g;
    }
    __syncthreads();
    const int nb = min(kTilePixels, len - b0);
    for (int jj = 0; jj < nb; ++jj) {
      const int pos = len - 1 - (b0 + jj);
      S g[12];
#pragma unroll
      for (int q = 0; q < 12; ++q) g[q] = S(0);
      bool took = false;
      if (inside && pos < lim) {
        const Staged<S> sp = s_sp[jj];
        Eval<S> e;
        ++evals;
        if (Ru::eval(sp, pxf, pyf, e)) {
          const S oma = S(1) - e.alpha;
          const S Tb = Tcur / oma;  // T in front of this splat
          const S dot = G0 * (sp.cr - acc0) + G1 * (sp.cg - acc1) + G2 * (sp.cb - acc2);
          acc0 = e.alpha * sp.cr + oma * acc0;
          acc1 = e.alpha * sp.cg + oma * acc1;
          acc2 = e.alpha * sp.cb + oma * acc2;
          Tcur = Tb;
          S dLda = Tb * dot;
          if constexpr (Ru::kBackground) dLda += (-T_final / oma) * bg_dot;
          const S w = e.alpha * Tb;
          g[6] = w * G0;
          g[7] = w * G1;
          g[8] = w * G2;
          shape_grads<R, S>(sp, e, dLda, g);
          if constexpr (R == kRulesPhase0) g[5] = g[5] * sp.o * (S(1) - sp.o);
          took = true;
        }
      }
      if constexpr (kPreReduce) {
        // the wavefront's pixels' gradients of the splat summed first (all lanes take the same
        // list entry), then one atomic per value from its owner lane
        if (__ballot(took ? 1 : 0) == 0) continue;  // wave-uniform
        S u0, u1;
        wave_reduce12(g, u0, u1);
        if (owner) atomic_add_grad(a.grad_rec + static_cast<int64_t>(s_id[jj]) * kGrad2D + kidx, lo == 0 ? u0 : u1);
        atomics += 9;
      } else {
        if (!took) continue;
        S* dst = a.grad_rec + static_cast<int64_t>(s_id[jj]) * kGrad2D;
#pragma unroll
        for (int q = 0; q < 9; ++q) atomic_add_grad(dst + q, g[q]);
        atomics += 9;
      }
    }
  }
  if (a.counters) {
    count_add(a.counters, atomics);
    count_add(a.counters + 2, evals);
  }
}

}  // namespace gs

using namespace gs;

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------
namespace {

template <int R, typename S>
void launch_fwd(const BlendArgs<S>& a, hipStream_t st) {
  if constexpr (R == kRules3D && std::is_same<S, float>::value) {
    // (the 3D forward takes no counters) one pixel per lane, a wavefront per strip, measured
    // fastest: 114 us at 1M SH3 against 118 with two and 165 with four (a wavefront per tile:
    // too few wavefronts, and the heaviest tiles run alone), and 120 for the shared-staging
    // blend_fwd_kernel
    constexpr int P = 1;
    constexpr int kTPB = 4 / (kStrips / P);
    hipLaunchKernelGGL(blend_fwd_strip_kernel<P>, dim3(static_cast<unsigned>((a.n_tiles + kTPB - 1) / kTPB)),
                       dim3(4 * kWave), 0, st, a);
  } else if (a.counters) {
    hipLaunchKernelGGL((blend_fwd_kernel<R, S, true>), dim3(a.n_tiles), dim3(kTilePixels), 0, st, a);
  } else {
    hipLaunchKernelGGL((blend_fwd_kernel<R, S, false>), dim3(a.n_tiles), dim3(kTilePixels), 0, st, a);
  }
}

// Workgroups (of one wavefront: 3D) of the striding list-driven backward: every CU holds its
// share several times over. Bucket tables longer than kBwdStrideFrom use it.
constexpr int64_t kBwdListBlocks = 256 * 64;
constexpr int64_t kBwdStrideFrom = 4 * kBwdListBlocks * 4;

template <int R, typename S, bool kCount, bool kAbs>
void launch_bwd_bucket_k(const BlendArgs<S>& a, hipStream_t st) {
  constexpr int kBwdWaves = bwd_waves<R>();
  int64_t blocks = (a.n_buckets + kBwdWaves - 1) / kBwdWaves;
  // (the walks' XCD runs map workgroups onto entries within whole groups of 8 kXcdRun)
  if (kBwdWaves == 1) blocks = (blocks + 8 * kXcdRun - 1) / (8 * kXcdRun) * (8 * kXcdRun);
  const dim3 block(kBwdWaves * kWave);
  if (a.bucket_list && blocks > kBwdStrideFrom)
    hipLaunchKernelGGL((blend_bwd_bucket_kernel<R, S, kCount, kAbs, 2>), dim3(static_cast<unsigned>(kBwdListBlocks)),
                       block, 0, st, a);
  else if (a.bucket_list)
    hipLaunchKernelGGL((blend_bwd_bucket_kernel<R, S, kCount, kAbs, 1>), dim3(static_cast<unsigned>(blocks)), block,
                       0, st, a);
  else
    hipLaunchKernelGGL((blend_bwd_bucket_kernel<R, S, kCount, kAbs, 0>), dim3(static_cast<unsigned>(blocks)), block,
                       0, st, a);
}

template <int R, typename S, bool kAbs = true>
void launch_bwd_bucket(const BlendArgs<S>& a, hipStream_t st) {
  if (a.counters)
    launch_bwd_bucket_k<R, S, true, kAbs>(a, st);
  else
    launch_bwd_bucket_k<R, S, false, kAbs>(a, st);
}

template <int R, typename S>
void launch_bwd_pixel(const BlendArgs<S>& a, hipStream_t st) {
  hipLaunchKernelGGL((blend_bwd_pixel_kernel<R, S>), dim3(a.n_tiles), dim3(kTilePixels), 0, st, a);
}

int check_rules(int rules, int dtype) {
  GS_REQUIRE(rules == GS_RULES_TOY2D || rules == GS_RULES_PHASE0, GS_ERR_ARG,
             "rules must be GS_RULES_TOY2D or GS_RULES_PHASE0 (got %d)", rules);
  GS_REQUIRE(dtype == GS_FLOAT32 || dtype == GS_FLOAT64, GS_ERR_ARG,
             "dtype must be GS_FLOAT32 or GS_FLOAT64 (got %d)", dtype);
  return GS_OK;
}

template <typename S>
BlendArgs<S> make_args(const void* rec, const uint32_t* ranges, int range_stride,
                       const uint32_t* point_list, const uint32_t* bucket_offsets, int W, int H,
                       const double* bg) {
  BlendArgs<S> a{};
  a.rec = static_cast<const S*>(rec);
  a.ranges = ranges;
  a.range_stride = range_stride;
  a.point_list = point_list;
  a.bucket_offsets = bucket_offsets;
  a.W = W;
  a.H = H;
  a.tiles_x = (W + kTile - 1) / kTile;
  a.n_tiles = a.tiles_x * ((H + kTile - 1) / kTile);
  a.bg0 = bg ? static_cast<S>(bg[0]) : S(0);
  a.bg1 = bg ? static_cast<S>(bg[1]) : S(0);
  a.bg2 = bg ? static_cast<S>(bg[2]) : S(0);
  return a;
}

template <typename F>
void dispatch2d(int rules, int dtype, F&& f) {
  if (rules == GS_RULES_TOY2D) {
    if (dtype == GS_FLOAT32) f(std::integral_constant<int, kRulesToy2D>{}, float{});
    else f(std::integral_constant<int, kRulesToy2D>{}, double{});
  } else {
    if (dtype == GS_FLOAT32) f(std::integral_constant<int, kRulesPhase0>{}, float{});
    else f(std::integral_constant<int, kRulesPhase0>{}, double{});
  }
}

}  // namespace

extern "C" int gs_blend_fwd_3d(const float* splat_rec, const uint32_t* ranges,
                               const uint32_t* point_list, const uint32_t* bucket_offsets,
                               int width, int height, const float* bg, float* image,
                               float* final_T, float* alpha, int32_t* n_contrib, uint32_t* tile_max,
                               float* ckpt, uint32_t* bucket_list, uint32_t* bucket_to_tile,
                               float* clear, int64_t clear_floats, int flags, void* stream) {
  clear_error();
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARG, "image size must be positive");
  GS_REQUIRE(clear_floats >= 0 && clear_floats % 4 == 0 && (clear || clear_floats == 0), GS_ERR_ARG,
             "clear must hold a multiple of 4 floats");
  GS_REQUIRE(aligned(clear, 16), GS_ERR_ALIGN, "clear must be 16-byte aligned");
  GS_REQUIRE(!bucket_to_tile || bucket_offsets, GS_ERR_ARG, "bucket_to_tile needs bucket_offsets");
  // splat_rec, point_list and ckpt may be NULL when the scene has no instances; without ckpt
  // (inference) bucket_offsets, n_contrib and tile_max may be NULL as well
  GS_REQUIRE(ranges && image && final_T && (!ckpt || (bucket_offsets && n_contrib && tile_max)), GS_ERR_ARG,
             "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16) && aligned(ckpt, 16), GS_ERR_ALIGN,
             "splat_rec and ckpt must be 16-byte aligned");
  const double bgd[3] = {bg ? bg[0] : 0.0, bg ? bg[1] : 0.0, bg ? bg[2] : 0.0};
  BlendArgs<float> a = make_args<float>(splat_rec, ranges, 2, point_list, bucket_offsets, width, height, bgd);
  a.image = image;
  a.final_T = final_T;
  a.alpha_out = alpha;
  a.n_contrib = n_contrib;
  a.tile_max = tile_max;
  a.ckpt = ckpt;
  GS_REQUIRE(!bucket_list || ckpt, GS_ERR_ARG, "bucket_list needs the checkpoints");
  GS_REQUIRE(aligned(bucket_list, 16), GS_ERR_ALIGN, "bucket_list must be 16-byte aligned");
  a.bucket_list = bucket_list;
  a.b2t_out = bucket_to_tile;
  a.clear4 = clear_floats ? reinterpret_cast<float4*>(clear) : nullptr;
  a.clear4_n = clear_floats / 4;
  if (bucket_list && !(flags & GS_BLEND_LIST_CLEARED))
    fill_zero_f32(reinterpret_cast<float*>(bucket_list), kListHeader, as_stream(stream));
  launch_fwd<kRules3D, float>(a, as_stream(stream));
  return check_launch("blend_fwd_3d");
}

extern "C" int gs_blend_scores_3d(const float* splat_rec, const uint32_t* ranges,
                                  const uint32_t* point_list, int width, int height, int64_t n,
                                  float* scores, void* stream) {
  clear_error();
  GS_REQUIRE(width > 0 && height > 0 && n >= 0, GS_ERR_ARG, "invalid sizes");
  GS_REQUIRE(ranges && (scores || n == 0), GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16), GS_ERR_ALIGN, "splat_rec must be 16-byte aligned");
  const double bgd[3] = {0.0, 0.0, 0.0};
  BlendArgs<float> a = make_args<float>(splat_rec, ranges, 2, point_list, nullptr, width, height, bgd);
  a.scores = scores;
  hipLaunchKernelGGL((blend_fwd_kernel<kRules3D, float, false, true>), dim3(a.n_tiles), dim3(kTilePixels), 0,
                     as_stream(stream), a);
  return check_launch("blend_scores_3d");
}

extern "C" int gs_blend_bwd_3d(const float* splat_rec, const uint32_t* ranges,
                               const uint32_t* point_list, const uint32_t* bucket_offsets,
                               const uint32_t* bucket_to_tile, int64_t n_buckets_max, int64_t n,
                               int width, int height, const float* image, const float* grad_image,
                               const float* final_T, const float* grad_alpha,
                               const int32_t* n_contrib, const uint32_t* tile_max,
                               const float* ckpt, uint32_t* bucket_list, float* grad2d,
                               double* grad_conic64, int flags, unsigned long long* counters,
                               void* stream) {
  clear_error();
  GS_REQUIRE(width > 0 && height > 0 && n >= 0 && n_buckets_max >= 0, GS_ERR_ARG,
             "invalid sizes");
  GS_REQUIRE(grad2d || n == 0, GS_ERR_ARG, "null grad2d");
  GS_REQUIRE(aligned(grad_conic64, 8), GS_ERR_ALIGN, "grad_conic64 must be 8-byte aligned");
  hipStream_t st = as_stream(stream);
  if (!(flags & GS_ACCUMULATE)) {
    fill_zero_f32(grad2d, n * kGrad2D, st);
    if (grad_conic64) fill_zero_f32(reinterpret_cast<float*>(grad_conic64), n * 8, st);
    if (int e = check_launch("blend_bwd_3d (zero fill)")) return e;
  }
  if (n_buckets_max == 0 || n == 0) return GS_OK;
  // splat_rec, point_list and ckpt may be NULL when there are no instances (no bucket reads them)
  GS_REQUIRE(ranges && bucket_offsets && bucket_to_tile && image && grad_image && n_contrib &&
                 tile_max && (final_T || !grad_alpha),
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16) && aligned(ckpt, 16), GS_ERR_ALIGN,
             "splat_rec and ckpt must be 16-byte aligned");
  BlendArgs<float> a = make_args<float>(splat_rec, ranges, 2, point_list, bucket_offsets, width, height, nullptr);
  a.image = const_cast<float*>(image);
  a.final_T = const_cast<float*>(final_T);
  a.n_contrib = const_cast<int32_t*>(n_contrib);
  a.tile_max = const_cast<uint32_t*>(tile_max);
  a.ckpt = const_cast<float*>(ckpt);
  a.bucket_to_tile = bucket_to_tile;
  a.n_buckets_dev = bucket_offsets + a.n_tiles;
  a.n_buckets = n_buckets_max;
  a.grad_image = grad_image;
  a.grad_alpha = grad_alpha;
  a.grad_rec = grad2d;
  a.conic64 = grad_conic64;
  a.counters = counters;
  GS_REQUIRE(aligned(bucket_list, 16), GS_ERR_ALIGN, "bucket_list must be 16-byte aligned");
  a.bucket_list = bucket_list;
  if (flags & GS_ABS_GRAD)
    launch_bwd_bucket<kRules3D, float, true>(a, st);
  else
    launch_bwd_bucket<kRules3D, float, false>(a, st);
  return check_launch("blend_bwd_3d");
}

extern "C" int gs2d_blend_fwd(int rules, int dtype, const void* rec, const uint32_t* ranges,
                              int range_stride, const uint32_t* point_list,
                              const uint32_t* bucket_offsets, int width, int height,
                              const double* bg, void* image, void* final_T, int32_t* n_contrib,
                              int32_t* last_contrib, uint32_t* tile_max, void* ckpt,
                              unsigned long long* counters, void* stream) {
  clear_error();
  if (int e = check_rules(rules, dtype)) return e;
  GS_REQUIRE(width > 0 && height > 0 && (range_stride == 1 || range_stride == 2), GS_ERR_ARG,
             "invalid image size or range stride");
  GS_REQUIRE(ranges && image && final_T && n_contrib && (bucket_offsets || !ckpt), GS_ERR_ARG,
             "null pointer argument");
  GS_REQUIRE(aligned(rec, 16) && aligned(ckpt, 16), GS_ERR_ALIGN, "rec and ckpt must be 16-byte aligned");
  int rc = GS_OK;
  dispatch2d(rules, dtype, [&](auto rr, auto s) {
    using S = decltype(s);
    constexpr int R = decltype(rr)::value;
    BlendArgs<S> a = make_args<S>(rec, ranges, range_stride, point_list, bucket_offsets, width, height, bg);
    a.image = static_cast<S*>(image);
    a.final_T = static_cast<S*>(final_T);
    a.n_contrib = n_contrib;
    a.last_contrib = last_contrib;
    a.tile_max = tile_max;
    a.ckpt = static_cast<S*>(ckpt);
    a.counters = counters;
    launch_fwd<R, S>(a, as_stream(stream));
    rc = check_launch("gs2d_blend_fwd");
  });
  return rc;
}

extern "C" int gs2d_blend_bwd_bucket(int rules, int dtype, const void* rec, const uint32_t* ranges,
                                     int range_stride, const uint32_t* point_list,
                                     const uint32_t* bucket_offsets, const uint32_t* bucket_to_tile,
                                     int64_t n_buckets, int64_t n, int width, int height,
                                     const void* image, const void* grad_image, const int32_t* limit,
                                     const uint32_t* tile_max, const void* ckpt, void* grad_rec,
                                     unsigned long long* counters, void* stream) {
  clear_error();
  if (int e = check_rules(rules, dtype)) return e;
  GS_REQUIRE(width > 0 && height > 0 && n >= 0 && n_buckets >= 0 &&
                 (range_stride == 1 || range_stride == 2),
             GS_ERR_ARG, "invalid sizes");
  GS_REQUIRE(grad_rec || n == 0, GS_ERR_ARG, "null grad_rec");
  hipStream_t st = as_stream(stream);
  const size_t esz = dtype == GS_FLOAT64 ? 8 : 4;
  if (n > 0) fill_zero_f32(static_cast<float*>(grad_rec), n * kGrad2D * static_cast<int64_t>(esz / 4), st);
  if (int e = check_launch("gs2d_blend_bwd_bucket (zero fill)")) return e;
  if (n_buckets == 0 || n == 0) return GS_OK;
  GS_REQUIRE(rec && ranges && point_list && bucket_offsets && bucket_to_tile && image && grad_image && ckpt &&
                 (limit || rules == GS_RULES_PHASE0),
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(rec, 16) && aligned(ckpt, 16), GS_ERR_ALIGN, "rec and ckpt must be 16-byte aligned");
  int rc = GS_OK;
  dispatch2d(rules, dtype, [&](auto rr, auto s) {
    using S = decltype(s);
    constexpr int R = decltype(rr)::value;
    BlendArgs<S> a = make_args<S>(rec, ranges, range_stride, point_list, bucket_offsets, width, height, nullptr);
    a.image = const_cast<S*>(static_cast<const S*>(image));
    a.n_contrib = const_cast<int32_t*>(limit);
    a.tile_max = const_cast<uint32_t*>(tile_max);
    a.ckpt = const_cast<S*>(static_cast<const S*>(ckpt));
    a.counters = counters;
    a.bucket_to_tile = bucket_to_tile;
    a.n_buckets = n_buckets;
    a.grad_image = static_cast<const S*>(grad_image);
    a.grad_rec = static_cast<S*>(grad_rec);
    launch_bwd_bucket<R, S>(a, st);
    rc = check_launch("gs2d_blend_bwd_bucket");
  });
  return rc;
}

extern "C" int gs2d_blend_bwd_pixel(int rules, int dtype, const void* rec, const uint32_t* ranges,
                                    int range_stride, const uint32_t* point_list, int64_t n,
                                    int width, int height, const double* bg, const void* final_T,
                                    const int32_t* limit, const void* grad_image, void* grad_rec,
                                    unsigned long long* counters, void* stream) {
  clear_error();
  if (int e = check_rules(rules, dtype)) return e;
  GS_REQUIRE(width > 0 && height > 0 && n >= 0 && (range_stride == 1 || range_stride == 2),
             GS_ERR_ARG, "invalid sizes");
  GS_REQUIRE(grad_rec || n == 0, GS_ERR_ARG, "null grad_rec");
  hipStream_t st = as_stream(stream);
  const size_t esz = dtype == GS_FLOAT64 ? 8 : 4;
  if (n > 0) fill_zero_f32(static_cast<float*>(grad_rec), n * kGrad2D * static_cast<int64_t>(esz / 4), st);
  if (int e = check_launch("gs2d_blend_bwd_pixel (zero fill)")) return e;
  if (n == 0) return GS_OK;
  GS_REQUIRE(rec && ranges && point_list && final_T && limit && grad_image, GS_ERR_ARG,
             "null pointer argument");
  GS_REQUIRE(aligned(rec, 16), GS_ERR_ALIGN, "rec must be 16-byte aligned");
  int rc = GS_OK;
  dispatch2d(rules, dtype, [&](auto rr, auto s) {
    using S = decltype(s);
    constexpr int R = decltype(rr)::value;
    BlendArgs<S> a = make_args<S>(rec, ranges, range_stride, point_list, nullptr, width, height, bg);
    a.final_T = const_cast<S*>(static_cast<const S*>(final_T));
    a.n_contrib = const_cast<int32_t*>(limit);
    a.counters = counters;
    a.grad_image = static_cast<const S*>(grad_image);
    a.grad_rec = static_cast<S*>(grad_rec);
    launch_bwd_pixel<R, S>(a, st);
    rc = check_launch("gs2d_blend_bwd_pixel");
  });
  return rc;
}
