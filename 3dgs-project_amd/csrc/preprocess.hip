// 3D preprocess, forward and backward.
//
// One thread per Gaussian, 256-thread workgroups. A wavefront's 64 Gaussians own one
// contiguous block of the [n, K, 3] SH tensor (64 * 3K floats); the wavefront moves that
// block through LDS with coalesced loads/stores (rows padded to an odd stride, so a lane's
// row reads are bank-conflict free), instead of each lane streaming its own 3K floats 3K * 4
// bytes apart. Degree-3 rows (48 floats) go through 32 rows at a time (each pass one
// contiguous block), which halves the LDS per wavefront and doubles the wavefronts a CU can
// hold. Same idea as the
// reference's coalesced SH access (phase2/sh_coalesce.patch:20-170,
// upstream/upstream_main_kernels.patch:26-76).
#include <stdarg.h>

#include "gs_host.h"
#include "gs_sh.h"

namespace gs {

// SH rows staged through LDS at a time: degree 3 in two passes of 32 rows (each pass one
// contiguous 6 KB block of the tensor), lower degrees in one pass of 64.
template <int K>
struct ShStage {
  static constexpr int R = 3 * K;            // floats per Gaussian row
  static constexpr int RH = K > 9 ? 32 : 64;  // rows per pass
  static constexpr int NH = 64 / RH;         // passes
  // Padded LDS row. Rows of whole float4s (degrees 1 and 3) take an odd number of float4s and
  // are moved with 16-byte LDS accesses (lanes reading their own rows hit distinct banks);
  // other rows take an odd number of floats (4-byte accesses, conflict-free the same way).
  static constexpr bool kVec = R % 4 == 0;
  static constexpr int CP = kVec ? 4 * ((R / 4) | 1) : (R | 1);
};

// SH coefficients of the Gaussians: one [n, K, 3] array, or (split) the DC [n, 1, 3] and the
// rest [n, K - 1, 3] as two arrays, the layout of trainers that give the two their own
// learning rates.
struct ShPtr {
  const float* a;  // [n, K, 3], or the DC [n, 1, 3] when b is set
  const float* b;  // the rest [n, K - 1, 3], or NULL
};
struct ShOut {
  float* a;
  float* b;
};

// rows x RW floats at blk (contiguous) -> LDS rows of pitch CP from column c0 (RW, CP fixed;
// FULL rows, if not 0: the unrolled path for a whole pass, every load in flight before the
// first store). Only the rows whose bit is set in `need` (bit r: row r) are read: the LDS rows
// of the others keep whatever they held.
template <int RW, int CP, int FULL>
__device__ __forceinline__ void rows_to_lds(const float* __restrict__ blk, int nr, float* srow, int c0, int lane,
                                            uint64_t need) {
  if constexpr (RW > 0) {
    constexpr int N4 = FULL * RW / 4;
    if constexpr (FULL > 0 && (FULL * RW) % 4 == 0 && RW % 4 == 0) {
      if (nr == FULL && aligned16(blk)) {
        constexpr int IT = (N4 + 63) / 64;
        float4 v[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int f4 = lane + 64 * it;
          if ((N4 % 64 == 0 || f4 < N4) && ((need >> (f4 / (RW / 4))) & 1u))
            v[it] = reinterpret_cast<const float4*>(blk)[f4];
        }
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int f4 = lane + 64 * it;
          if ((N4 % 64 == 0 || f4 < N4) && ((need >> (f4 / (RW / 4))) & 1u)) {
            // a float4 never crosses a row
            const int row = f4 / (RW / 4), q = f4 - row * (RW / 4);
            float* d = srow + row * CP + c0 + 4 * q;
            if (CP % 4 == 0 && c0 == 0) {
              *reinterpret_cast<float4*>(d) = make_float4(v[it].x, v[it].y, v[it].z, v[it].w);
            } else {
              d[0] = v[it].x; d[1] = v[it].y; d[2] = v[it].z; d[3] = v[it].w;
            }
          }
        }
        return;
      }
    }
    const int total = nr * RW;
    if (aligned16(blk)) {
      const int n4 = total >> 2;
      for (int f4 = lane; f4 < n4; f4 += 64) {
        // a float4 of rows not a multiple of 4 floats long can span two rows: read it if either
        // is needed
        const int r0 = (4 * f4) / RW, r1 = (4 * f4 + 3) / RW;
        if ((((need >> r0) | (need >> r1)) & 1u) == 0u) continue;
        const float4 v = reinterpret_cast<const float4*>(blk)[f4];
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int idx = 4 * f4 + e, row = idx / RW;
          srow[row * CP + c0 + idx - row * RW] = vv[e];
        }
      }
      for (int idx = 4 * n4 + lane; idx < total; idx += 64) {
        const int row = idx / RW;
        if ((need >> row) & 1u) srow[row * CP + c0 + idx - row * RW] = blk[idx];
      }
    } else {
      for (int idx = lane; idx < total; idx += 64) {
        const int row = idx / RW;
        if ((need >> row) & 1u) srow[row * CP + c0 + idx - row * RW] = blk[idx];
      }
    }
  }
}

template <int RW, int CP>
__device__ __forceinline__ void lds_to_rows(float* __restrict__ blk, int nr, const float* srow, int c0, int lane) {
  if constexpr (RW > 0) {
    const int total = nr * RW;
    if (aligned16(blk)) {
      const int n4 = total >> 2;
      for (int f4 = lane; f4 < n4; f4 += 64) {
        float vv[4];
        if constexpr (RW % 4 == 0) {  // a float4 never crosses a row
          const int row = f4 / (RW / 4), q = f4 - row * (RW / 4);
          const float* d = srow + row * CP + c0 + 4 * q;
          if (CP % 4 == 0 && c0 == 0) {
            const float4 v = *reinterpret_cast<const float4*>(d);
            vv[0] = v.x; vv[1] = v.y; vv[2] = v.z; vv[3] = v.w;
          } else {
            vv[0] = d[0]; vv[1] = d[1]; vv[2] = d[2]; vv[3] = d[3];
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int idx = 4 * f4 + e, row = idx / RW;
            vv[e] = srow[row * CP + c0 + idx - row * RW];
          }
        }
        reinterpret_cast<float4*>(blk)[f4] = make_float4(vv[0], vv[1], vv[2], vv[3]);
      }
      for (int idx = 4 * n4 + lane; idx < total; idx += 64) {
        const int row = idx / RW;
        blk[idx] = srow[row * CP + c0 + idx - row * RW];
      }
    } else {
      for (int idx = lane; idx < total; idx += 64) {
        const int row = idx / RW;
        blk[idx] = srow[row * CP + c0 + idx - row * RW];
      }
    }
  }
}

// Copies rows [RH h, RH h + RH) of the wavefront's `rows` SH rows (the wavefront's first row is
// `first`) into LDS rows of stride CP; only the rows of the Gaussians set in `vmask` (bit l:
// the wavefront's Gaussian l) are read from memory.
template <int K>
__device__ __forceinline__ void stage_sh(ShPtr src, int64_t first, int rows, int h, float* srow, int lane,
                                         uint64_t vmask) {
  using St = ShStage<K>;
  constexpr int R = St::R, CP = St::CP, RH = St::RH;
  const int r0 = RH * h;
  const int nr = min(RH, rows - r0);
  if (nr <= 0) return;
  const int64_t row = first + r0;
  const uint64_t need = vmask >> r0;
  if (src.b == nullptr) {
    rows_to_lds<R, CP, RH>(src.a + row * R, nr, srow, 0, lane, need);
  } else {
    // (the split layout takes the plain loop: an unrolled one for rows not a multiple of four
    // floats costs the kernel registers, i.e. occupancy, on the single-array path too)
    rows_to_lds<3, CP, 0>(src.a + row * 3, nr, srow, 0, lane, need);
    rows_to_lds<R - 3, CP, 0>(src.b + row * (R - 3), nr, srow, 3, lane, need);
  }
}

// Register copy of one pass of a full wavefront's SH rows (single-array layout, rows whose
// float count is a multiple of 4: degrees 1 and 3), so that a pass's loads can be issued long
// before its rows go to LDS. load() and store() take the same `need` (bit r: the pass's row r).
template <int K>
struct ShPrefetch {
  using St = ShStage<K>;
  static constexpr int R = St::R, RH = St::RH, CP = St::CP;
  static constexpr bool kOk = R % 4 == 0;
  static constexpr int N4 = RH * R / 4;  // float4 per pass
  static constexpr int IT = (N4 + 63) / 64;
  float4 v[kOk ? IT : 1];

  __device__ __forceinline__ static bool row_needed(int f4, uint64_t need) {
    return (N4 % 64 == 0 || f4 < N4) && ((need >> (f4 / (R / 4))) & 1u);
  }
  // blk: the pass's first row
  __device__ __forceinline__ void load(const float* __restrict__ blk, uint64_t need, int lane) {
    if constexpr (kOk) {
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int f4 = lane + 64 * it;
        if (row_needed(f4, need)) v[it] = reinterpret_cast<const float4*>(blk)[f4];
      }
    }
  }
  __device__ __forceinline__ void store(float* srow, uint64_t need, int lane) const {
    if constexpr (kOk) {
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int f4 = lane + 64 * it;
        if (row_needed(f4, need)) {  // a float4 never crosses a row
          const int row = f4 / (R / 4), q = f4 - row * (R / 4);
          // (CP % 4 == 0 for these rows; the float4 rebuilt from its parts keeps v in registers)
          *reinterpret_cast<float4*>(srow + row * CP + 4 * q) = make_float4(v[it].x, v[it].y, v[it].z, v[it].w);
        }
      }
    }
  }
};

// Writes the staged rows of pass h back to the wavefront's rows.
template <int K>
__device__ __forceinline__ void unstage_sh(ShOut dst, int64_t first, int rows, int h, const float* srow, int lane) {
  using St = ShStage<K>;
  constexpr int R = St::R, CP = St::CP, RH = St::RH;
  const int r0 = RH * h;
  const int nr = min(RH, rows - r0);
  if (nr <= 0) return;
  const int64_t row = first + r0;
  if (dst.b == nullptr) {
    lds_to_rows<R, CP>(dst.a + row * R, nr, srow, 0, lane);
  } else {
    lds_to_rows<3, CP>(dst.a + row * 3, nr, srow, 0, lane);
    lds_to_rows<R - 3, CP>(dst.b + row * (R - 3), nr, srow, 3, lane);
  }
}

struct Geom {
  bool vis;
  float vx, vy, vz, iz, tx, ty, txc, tyc;
  float o;                     // blended opacity (sigmoid, times rho under proper antialiasing)
  float os;                    // sigmoid of the opacity logit
  float rho, ratio;            // antialiasing compensation sqrt(ratio), ratio = det raw / det
  float qw, qx, qy, qz, qinv;  // normalised quaternion and 1/|q|
  float R[9];                  // rotation of the Gaussian
  float s[3];                  // scales
  float M[9];                  // R diag(s)
  float S[6];                  // 3D covariance (00 01 02 11 12 22)
  float T[6];                  // J W, 2x3
  float a, b, c;               // 2D covariance incl. dilation
  float ar, cr;                // diagonal of the 2D covariance without dilation
  float det, A, B, C;          // conic
  float mx, my;                // mean2d
};

// The forward geometry of one Gaussian. The operation order is part of the rule set: the
// CPU oracle evaluates the same sequence.
__device__ __forceinline__ void compute_geom(const float* __restrict__ means,
                                             const float* __restrict__ log_scales,
                                             const float4* __restrict__ quats,
                                             const float* __restrict__ opacity_logits,
                                             int64_t i, const CamK& cam, Geom& g) {
  const float px = means[3 * i], py = means[3 * i + 1], pz = means[3 * i + 2];
  g.vx = fmaf(cam.r[0], px, fmaf(cam.r[1], py, fmaf(cam.r[2], pz, cam.t[0])));
  g.vy = fmaf(cam.r[3], px, fmaf(cam.r[4], py, fmaf(cam.r[5], pz, cam.t[1])));
  g.vz = fmaf(cam.r[6], px, fmaf(cam.r[7], py, fmaf(cam.r[8], pz, cam.t[2])));
  bool vis = (g.vz > cam.znear) && (g.vz < cam.zfar);
  g.o = sigmoid(opacity_logits[i]);
  vis = vis && (g.o >= kAlphaMin);

  const float4 q = quats[i];
  const float n2 = fmaf(q.x, q.x, fmaf(q.y, q.y, fmaf(q.z, q.z, q.w * q.w)));
  vis = vis && (n2 > 0.0f);
  g.qinv = 1.0f / sqrtf(n2);
  const float w = q.x * g.qinv, x = q.y * g.qinv, y = q.z * g.qinv, z = q.w * g.qinv;
  g.qw = w;
  g.qx = x;
  g.qy = y;
  g.qz = z;
  const float xx = x * x, yy = y * y, zz = z * z;
  const float xy = x * y, xz = x * z, yz = y * z;
  const float wx = w * x, wy = w * y, wz = w * z;
  float t;
  t = yy + zz; t = t + t; g.R[0] = 1.0f - t;
  t = xy - wz; g.R[1] = t + t;
  t = xz + wy; g.R[2] = t + t;
  t = xy + wz; g.R[3] = t + t;
  t = xx + zz; t = t + t; g.R[4] = 1.0f - t;
  t = yz - wx; g.R[5] = t + t;
  t = xz - wy; g.R[6] = t + t;
  t = yz + wx; g.R[7] = t + t;
  t = xx + yy; t = t + t; g.R[8] = 1.0f - t;

  for (int k = 0; k < 3; ++k) g.s[k] = exp_any(log_scales[3 * i + k]);
  for (int r = 0; r < 3; ++r)
    for (int k = 0; k < 3; ++k) g.M[3 * r + k] = g.R[3 * r + k] * g.s[k];
  const float* M = g.M;
  g.S[0] = fmaf(M[0], M[0], fmaf(M[1], M[1], M[2] * M[2]));
  g.S[1] = fmaf(M[0], M[3], fmaf(M[1], M[4], M[2] * M[5]));
  g.S[2] = fmaf(M[0], M[6], fmaf(M[1], M[7], M[2] * M[8]));
  g.S[3] = fmaf(M[3], M[3], fmaf(M[4], M[4], M[5] * M[5]));
  g.S[4] = fmaf(M[3], M[6], fmaf(M[4], M[7], M[5] * M[8]));
  g.S[5] = fmaf(M[6], M[6], fmaf(M[7], M[7], M[8] * M[8]));

  g.iz = 1.0f / g.vz;
  g.tx = g.vx * g.iz;
  g.ty = g.vy * g.iz;
  g.txc = fminf(fmaxf(g.tx, cam.lim_x_lo), cam.lim_x_hi);
  g.tyc = fminf(fmaxf(g.ty, cam.lim_y_lo), cam.lim_y_hi);
  const float j00 = cam.fx * g.iz, j11 = cam.fy * g.iz;
  const float j02 = -(j00 * g.txc), j12 = -(j11 * g.tyc);
  for (int k = 0; k < 3; ++k) {
    g.T[k] = fmaf(j00, cam.r[k], j02 * cam.r[6 + k]);
    g.T[3 + k] = fmaf(j11, cam.r[3 + k], j12 * cam.r[6 + k]);
  }
  const float* S = g.S;
  const float* T = g.T;
  // U = T S (2x3), S symmetric with rows (S0 S1 S2), (S1 S3 S4), (S2 S4 S5)
  const float u00 = fmaf(T[0], S[0], fmaf(T[1], S[1], T[2] * S[2]));
  const float u01 = fmaf(T[0], S[1], fmaf(T[1], S[3], T[2] * S[4]));
  const float u02 = fmaf(T[0], S[2], fmaf(T[1], S[4], T[2] * S[5]));
  const float u10 = fmaf(T[3], S[0], fmaf(T[4], S[1], T[5] * S[2]));
  const float u11 = fmaf(T[3], S[1], fmaf(T[4], S[3], T[5] * S[4]));
  const float u12 = fmaf(T[3], S[2], fmaf(T[4], S[4], T[5] * S[5]));
  g.ar = fmaf(u00, T[0], fmaf(u01, T[1], u02 * T[2]));
  g.b = fmaf(u00, T[3], fmaf(u01, T[4], u02 * T[5]));
  g.cr = fmaf(u10, T[3], fmaf(u11, T[4], u12 * T[5]));
  g.a = g.ar + kDilation;
  g.c = g.cr + kDilation;
  g.det = fmaf(g.a, g.c, -(g.b * g.b));
  vis = vis && (g.det > 0.0f);
  g.os = g.o;
  g.rho = 1.0f;
  g.ratio = 1.0f;
  if (cam.flags & GS_CAM_PROPER_ANTIALIASING) {
    // opacity compensation of the 0.3 px^2 low-pass: o sqrt(det(S) / det(S + 0.3 I))
    const float det_raw = fmaf(g.ar, g.cr, -(g.b * g.b));
    g.ratio = fmaxf(det_raw / g.det, 0.0f);
    g.rho = sqrtf(g.ratio);
    g.o = g.os * g.rho;
    vis = vis && (g.o >= kAlphaMin);
  }
  const float idet = 1.0f / g.det;
  g.A = g.c * idet;
  g.B = -g.b * idet;
  g.C = g.a * idet;
  g.mx = fmaf(cam.fx, g.tx, cam.cx);
  g.my = fmaf(cam.fy, g.ty, cam.cy);
  g.vis = vis;
}

// acc[ch] = basis[0] row[ch] + sum over 0 < k < active of basis[k] row[3 k + ch] (fmaf, each
// channel's terms in k order) from the lane's LDS row; rows of whole float4s are read 16 bytes
// at a time (the same operations in the same order: the same bits).
template <int K>
__device__ __forceinline__ void sh_dot_row(const float* row, const float* basis, int active, float acc[3]) {
  using St = ShStage<K>;
  if constexpr (St::kVec) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
    for (int c4 = 0; c4 < K / 4; ++c4) {  // 4 coefficients = 12 floats = 3 float4
      const float4 v0 = r4[3 * c4], v1 = r4[3 * c4 + 1], v2 = r4[3 * c4 + 2];
      const float c[4][3] = {{v0.x, v0.y, v0.z}, {v0.w, v1.x, v1.y}, {v1.z, v1.w, v2.x}, {v2.y, v2.z, v2.w}};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 4 * c4 + j;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
          if (k == 0) {
            acc[ch] = basis[0] * c[j][ch];
          } else {
            const float t = fmaf(basis[k], c[j][ch], acc[ch]);
            acc[ch] = k < active ? t : acc[ch];  // a select: no branches in the unrolled body
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
      acc[ch] = basis[0] * row[ch];
      for (int k = 1; k < active; ++k) acc[ch] = fmaf(basis[k], row[3 * k + ch], acc[ch]);
    }
  }
}

// Backward of the SH dot: gb[k] = row_k . gcol (the basis gradient) and the row overwritten
// with the coefficient gradients basis[k] gcol (zero for k >= active), read and written 16
// bytes at a time for rows of whole float4s.
template <int K>
__device__ __forceinline__ void sh_row_grads(float* row, const float* basis, int active, const float gcol[3],
                                             float* gb) {
  using St = ShStage<K>;
  if constexpr (St::kVec) {
    float4* r4 = reinterpret_cast<float4*>(row);
#pragma unroll
    for (int c4 = 0; c4 < K / 4; ++c4) {  // 4 coefficients = 12 floats = 3 float4
      if (c4) __builtin_amdgcn_sched_barrier(0);  // one chunk of row values live at a time
      const float4 v0 = r4[3 * c4], v1 = r4[3 * c4 + 1], v2 = r4[3 * c4 + 2];
      const int k = 4 * c4;
      const bool on0 = k < active, on1 = k + 1 < active, on2 = k + 2 < active, on3 = k + 3 < active;
      gb[k] = on0 ? v0.x * gcol[0] + v0.y * gcol[1] + v0.z * gcol[2] : 0.0f;
      gb[k + 1] = on1 ? v0.w * gcol[0] + v1.x * gcol[1] + v1.y * gcol[2] : 0.0f;
      gb[k + 2] = on2 ? v1.z * gcol[0] + v1.w * gcol[1] + v2.x * gcol[2] : 0.0f;
      gb[k + 3] = on3 ? v2.y * gcol[0] + v2.z * gcol[1] + v2.w * gcol[2] : 0.0f;
      const float b0 = on0 ? basis[k] : 0.0f, b1 = on1 ? basis[k + 1] : 0.0f;
      const float b2 = on2 ? basis[k + 2] : 0.0f, b3 = on3 ? basis[k + 3] : 0.0f;
      r4[3 * c4] = make_float4(b0 * gcol[0], b0 * gcol[1], b0 * gcol[2], b1 * gcol[0]);
      r4[3 * c4 + 1] = make_float4(b1 * gcol[1], b1 * gcol[2], b2 * gcol[0], b2 * gcol[1]);
      r4[3 * c4 + 2] = make_float4(b2 * gcol[2], b3 * gcol[0], b3 * gcol[1], b3 * gcol[2]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const bool on = k < active;
      gb[k] = on ? row[3 * k] * gcol[0] + row[3 * k + 1] * gcol[1] + row[3 * k + 2] * gcol[2] : 0.0f;
      const float bk = on ? basis[k] : 0.0f;
      row[3 * k] = bk * gcol[0];
      row[3 * k + 1] = bk * gcol[1];
      row[3 * k + 2] = bk * gcol[2];
    }
  }
}

template <int K>
__global__ __launch_bounds__(256) void preprocess_fwd_kernel(
    const float* __restrict__ means, const float* __restrict__ log_scales,
    const float4* __restrict__ quats, const float* __restrict__ opacity_logits,
    ShPtr sh, int64_t n, int active, CamK cam, SplatRec* __restrict__ rec,
    uint32_t* __restrict__ tiles_touched, uint32_t* __restrict__ depth_keys, uint32_t* __restrict__ wave_counts) {
  using St = ShStage<K>;
  // per wavefront: the tile-count scratch, then the SH rows
  constexpr int kWords = ((St::RH * St::CP > kCountScratchWords ? St::RH * St::CP : kCountScratchWords) + 3) & ~3;
  __shared__ __align__(16) float s_sh[4][kWords];  // each wavefront's rows 16-byte aligned
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * 256 + wave * 64;
  if (wave_first >= n) return;  // whole wavefront
  const int64_t i = wave_first + lane;
  const bool valid = i < n;

  Geom g;
  g.vis = false;
  int4 bnd = make_int4(0, -1, 0, -1);
  float thr = 0.0f;
  if (valid) {
    compute_geom(means, log_scales, quats, opacity_logits, i, cam, g);
    if (g.vis) {
      thr = log_pos(255.0f * g.o);
      const float t2 = thr + thr;
      const float ex = sqrtf(t2 * g.a), ey = sqrtf(t2 * g.c);
      float xf0 = ceilf((g.mx - ex) - 0.5f), xf1 = floorf((g.mx + ex) - 0.5f);
      float yf0 = ceilf((g.my - ey) - 0.5f), yf1 = floorf((g.my + ey) - 0.5f);
      bool ok = (thr > 0.0f) && __builtin_isfinite(xf0) && __builtin_isfinite(xf1) &&
                __builtin_isfinite(yf0) && __builtin_isfinite(yf1);
      xf0 = fmaxf(xf0, 0.0f);
      yf0 = fmaxf(yf0, 0.0f);
      xf1 = fminf(xf1, static_cast<float>(cam.width - 1));
      yf1 = fminf(yf1, static_cast<float>(cam.height - 1));
      ok = ok && (xf0 <= xf1) && (yf0 <= yf1);
      if (ok) {
        bnd = make_int4(static_cast<int>(xf0), static_cast<int>(xf1), static_cast<int>(yf0),
                        static_cast<int>(yf1));
      }
      g.vis = ok;
    }
  }
  float4 ra = make_float4(0.0f, 0.0f, 0.0f, 0.0f), rb = ra;
  if (g.vis) {
    ra = make_float4(g.mx, g.my, g.A, g.B);
    rb = make_float4(g.C, g.o, g.vz, thr);
  }
  // A full wavefront of the single SH array (degrees 1 and 3) issues its first pass's row loads
  // now, for the Gaussians visible so far (a superset of those with tiles), so that they are in
  // flight during the tile count and the SH basis; each later pass's loads go out as soon as
  // the previous pass is in LDS.
  const int rows = static_cast<int>(min<int64_t>(64, n - wave_first));
  const float* sh_blk = sh.a + wave_first * St::R;
  const bool prefetch = ShPrefetch<K>::kOk && sh.b == nullptr && rows == 64 && aligned16(sh_blk);
  const uint64_t pre_mask = __ballot(g.vis ? 1 : 0);
  ShPrefetch<K> pf;
  if (prefetch && pre_mask != 0) pf.load(sh_blk, pre_mask, lane);
  // tile rows of the wavefront's splats shared out over its lanes
  const uint32_t count = wave_count_rows(g.vis, ra, rb, bnd, lane, reinterpret_cast<uint32_t*>(s_sh[wave]));
  if (g.vis) g.vis = count > 0;

  // Colour: stage the wavefront's SH rows through LDS (wave-uniform branch).
  const uint64_t vmask = __ballot(g.vis ? 1 : 0);
  float col[3] = {0.0f, 0.0f, 0.0f};
  uint32_t mask = 0;
  if (vmask != 0) {
    float* srow = s_sh[wave];
    float basis[16];
    float acc[3] = {0.0f, 0.0f, 0.0f};
    if (g.vis) {
      const float dx = means[3 * i] - cam.campos[0];
      const float dy = means[3 * i + 1] - cam.campos[1];
      const float dz = means[3 * i + 2] - cam.campos[2];
      const float len = sqrtf(fmaf(dx, dx, fmaf(dy, dy, dz * dz)));
      const float il = 1.0f / len;
      sh_basis(dx * il, dy * il, dz * il, active, basis);
    }
#pragma unroll
    for (int h = 0; h < St::NH; ++h) {
      if (h) wave_sync();  // every lane is done with the previous rows
      if (prefetch) {
        const uint64_t need = pre_mask >> (St::RH * h);
        pf.store(srow, need, lane);
        if (h + 1 < St::NH) pf.load(sh_blk + St::RH * (h + 1) * St::R, pre_mask >> (St::RH * (h + 1)), lane);
      } else {
        stage_sh<K>(sh, wave_first, rows, h, srow, lane, vmask);
      }
      wave_sync();
      if (g.vis && lane / St::RH == h) {
        sh_dot_row<K>(srow + (lane - St::RH * h) * St::CP, basis, active, acc);
      }
    }
    if (g.vis) {
#pragma unroll
      for (int ch = 0; ch < 3; ++ch) {
        const float a = acc[ch] + 0.5f;
        if (a < 0.0f) mask |= (1u << ch);
        col[ch] = fmaxf(a, 0.0f);
      }
    }
  }
  if (valid) {
    tiles_touched[i] = g.vis ? count : 0u;
    // depth sort key: the orderable bits of the view depth, culled Gaussians last
    if (depth_keys) depth_keys[i] = g.vis ? float_order_key(rb.z) - cam.dkey0 : cam.dkey_cull;
    if (g.vis) {
      SplatRec r;
      r.a = ra;
      r.b = rb;
      r.c = make_float4(col[0], col[1], col[2], __uint_as_float(mask));
      r.d = bnd;
      rec[i] = r;
    } else {
      rec[i].d = make_int4(0, -1, 0, -1);  // empty bounds: the binning skips the record
    }
  }
  if (wave_counts) {
    // tiles touched by this wavefront's 64 Gaussians: the instance count m is their total
    uint32_t s = (valid && g.vis) ? count : 0u;
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) wave_counts[wave_first / 64] = s;
  }
}

// ---------------------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------------------
// Adds v = dL/dR[idx] (R row-major, the rotation of the unit quaternion (w, x, y, z)) to half the
// quaternion gradient: R[0] = 1 - 2(y^2 + z^2), R[1] = 2(xy - wz), R[2] = 2(xz + wy),
// R[3] = 2(xy + wz), R[4] = 1 - 2(x^2 + z^2), R[5] = 2(yz - wx), R[6] = 2(xz - wy),
// R[7] = 2(yz + wx), R[8] = 1 - 2(x^2 + y^2). idx is a compile-time constant after unrolling.
__device__ __forceinline__ void quat_grad_add(int idx, double v, double w, double x, double y, double z, double& gw,
                                              double& gx, double& gy, double& gz) {
  switch (idx) {
    case 0: gy -= 2.0 * y * v; gz -= 2.0 * z * v; break;
    case 1: gw -= z * v; gx += y * v; gy += x * v; gz -= w * v; break;
    case 2: gw += y * v; gx += z * v; gy += w * v; gz += x * v; break;
    case 3: gw += z * v; gx += y * v; gy += x * v; gz += w * v; break;
    case 4: gx -= 2.0 * x * v; gz -= 2.0 * z * v; break;
    case 5: gw -= x * v; gx -= w * v; gy += z * v; gz += y * v; break;
    case 6: gw -= y * v; gx += z * v; gy -= w * v; gz += x * v; break;
    case 7: gw += x * v; gx += w * v; gy += z * v; gz += y * v; break;
    default: gx -= 2.0 * x * v; gy -= 2.0 * y * v; break;
  }
}

// Wavefronts per workgroup of the preprocess backward: one (each takes its own 64 Gaussians and
// shares nothing with the others; 1M SH3: 105.5 -> 104.0 us against four per workgroup, while the
// forward, whose wavefronts are more alike, stays at four: 69.6 against 70.9 us with one).
constexpr int kPreBwdWaves = 1;
template <int K>
__global__ __launch_bounds__(kPreBwdWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void preprocess_bwd_kernel(
    const float* __restrict__ means, const float* __restrict__ log_scales,
    const float4* __restrict__ quats, const float* __restrict__ opacity_logits,
    ShPtr sh, int64_t n, int active, CamK cam, const uint32_t* __restrict__ tiles_touched,
    const float* __restrict__ grad2d, const double* __restrict__ conic64, float* __restrict__ g_means,
    float* __restrict__ g_log_scales, float4* __restrict__ g_quats,
    float* __restrict__ g_opacity, ShOut g_sh) {
  using St = ShStage<K>;
  __shared__ __align__(16) float s_sh[kPreBwdWaves][St::RH * St::CP];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * (kPreBwdWaves * 64) + wave * 64;
  if (wave_first >= n) return;
  const int64_t i = wave_first + lane;
  const bool valid = i < n;
  const bool vis = valid && tiles_touched[i] != 0u;
  const uint64_t vmask = __ballot(vis ? 1 : 0);
  float* srow = s_sh[wave];
  const int rows = static_cast<int>(min<int64_t>(64, n - wave_first));

  float gm[3] = {0.0f, 0.0f, 0.0f};  // dL/dmean (world)
  float gcol[3] = {0.0f, 0.0f, 0.0f};
  float gdl[3] = {0.0f, 0.0f, 0.0f};  // dL/dlog_scale
  float4 gq = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float gop = 0.0f;

  // ---- SH colour: coefficient gradients (through the LDS rows) and view-direction gradient ----
  const float* g2 = grad2d + i * kGrad2D;
  float dx = 0.0f, dy = 0.0f, dz = 0.0f, il = 0.0f;
  float basis[16], gb[16];
  if (vis) {
    const float dxw = means[3 * i] - cam.campos[0];
    const float dyw = means[3 * i + 1] - cam.campos[1];
    const float dzw = means[3 * i + 2] - cam.campos[2];
    const float len = sqrtf(fmaf(dxw, dxw, fmaf(dyw, dyw, dzw * dzw)));
    il = 1.0f / len;
    dx = dxw * il;
    dy = dyw * il;
    dz = dzw * il;
    sh_basis(dx, dy, dz, active, basis);
  }
#pragma unroll
  for (int h = 0; h < St::NH; ++h) {
    if (vmask != 0) {
      if (h) wave_sync();  // the previous rows are written out
      // (rows of culled Gaussians are not read: their lanes write zeros over them below)
      stage_sh<K>(sh, wave_first, rows, h, srow, lane, vmask);
      wave_sync();
      if (lane / St::RH == h) {
        float* row = srow + (lane - St::RH * h) * St::CP;
        if (vis) {
          // the forward's colour clamp (a channel clamped at 0 passes no gradient), recomputed
          // from the same rows and basis in the forward's operation order: the same bits, without
          // reading the 64-byte splat record for its mask
          float acc[3];
          sh_dot_row<K>(row, basis, active, acc);
#pragma unroll
          for (int ch = 0; ch < 3; ++ch) gcol[ch] = (acc[ch] + 0.5f < 0.0f) ? 0.0f : g2[6 + ch];
          // overwrite the row with the coefficient gradients (after its values were read)
          sh_row_grads<K>(row, basis, active, gcol, gb);
        } else if (valid) {
          if constexpr (St::kVec) {
            for (int q = 0; q < St::R / 4; ++q) reinterpret_cast<float4*>(row)[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          } else {
            for (int c = 0; c < St::R; ++c) row[c] = 0.0f;
          }
        }
      }
      wave_sync();
      unstage_sh<K>(g_sh, wave_first, rows, h, srow, lane);
    }
  }
  if (vmask == 0) {  // no visible Gaussian: zero rows
    if (g_sh.b == nullptr) {
      float* dst = g_sh.a + wave_first * St::R;
      for (int f = lane; f < rows * St::R; f += 64) dst[f] = 0.0f;
    } else {
      float* d0 = g_sh.a + wave_first * 3;
      float* d1 = g_sh.b + wave_first * (St::R - 3);
      for (int f = lane; f < rows * 3; f += 64) d0[f] = 0.0f;
      for (int f = lane; f < rows * (St::R - 3); f += 64) d1[f] = 0.0f;
    }
  }

  if (vis) {
    float gdx, gdy, gdz;
    sh_basis_grad(dx, dy, dz, active, gb, gdx, gdy, gdz);
    // d dir / d v = (I - d d^T) / |v|
    const float dd = dx * gdx + dy * gdy + dz * gdz;
    gm[0] = (gdx - dx * dd) * il;
    gm[1] = (gdy - dy * dd) * il;
    gm[2] = (gdz - dz * dd) * il;

    // ---- geometry: the forward's float32 intermediates (the same bits as the forward), the
    // chain rule in float64. The conic -> covariance step divides by det^2 and its terms cancel
    // for elongated splats (det << a c); in float32 such Gaussians get gradients off by more than
    // their own size. FP64 costs this memory-bound kernel nothing measurable. ----
    Geom g;
    compute_geom(means, log_scales, quats, opacity_logits, i, cam, g);
    const bool aa = cam.flags & GS_CAM_PROPER_ANTIALIASING;
    // grad2d[5] = sum alpha dL/dalpha = o dL/do for the blended opacity o (= os rho under proper
    // antialiasing); with o = sigmoid(logit) rho: dL/dlogit = dL/do rho os (1 - os) = g2[5] (1 - os)
    gop = static_cast<float>(static_cast<double>(g2[5]) * (1.0 - (aa ? g.os : g.o)));

    // mean2d = (fx vx/vz + cx, fy vy/vz + cy)
    const double fx = cam.fx, fy = cam.fy;
    const double iz = 1.0 / static_cast<double>(g.vz), iz2 = iz * iz;
    double gvx = g2[0] * fx * iz;
    double gvy = g2[1] * fy * iz;
    double gvz = -(g2[0] * fx * g.vx + g2[1] * fy * g.vy) * iz2;

    // conic (A, B, C) = (c, -b, a) / det  ->  2D covariance (a, b, c); a row marked by the blend
    // backward (slot 11) also has float64 conic sums (its elongated-splat buckets)
    double gA = g2[2], gB = g2[3], gC = g2[4];
    if (conic64 && g2[11] != 0.0f) {
      gA += conic64[4 * i];
      gB += conic64[4 * i + 1];
      gC += conic64[4 * i + 2];
    }
    const double a = g.a, b = g.b, c = g.c;
    const double det = a * c - b * b;
    const double id2 = 1.0 / (det * det);
    double ga = (-c * c * gA + b * c * gB - b * b * gC) * id2;
    double gbb = (2.0 * b * c * gA - (a * c + b * b) * gB + 2.0 * a * b * gC) * id2;
    double gc = (-b * b * gA + a * b * gB - a * a * gC) * id2;
    if (aa) {
      // rho^2 = (ar cr - b^2) / (a c - b^2), a = ar + 0.3, c = cr + 0.3:
      // d rho = d(rho^2) / (2 rho), d(rho^2)/da = (cr - rho^2 c) / det,
      // d(rho^2)/dc = (ar - rho^2 a) / det, d(rho^2)/db = -2 b (1 - rho^2) / det
      const double ar = g.ar, cr = g.cr;
      const double ratio = (ar * cr - b * b) / det;
      // dL/drho = dL/do os = g2[5] / rho, d rho = d ratio / (2 rho)
      const double k = static_cast<double>(g2[5]) / (2.0 * static_cast<double>(g.rho) * sqrt(ratio) * det);
      ga += k * (cr - ratio * c);
      gc += k * (ar - ratio * a);
      gbb += -2.0 * k * b * (1.0 - ratio);
    }
    // cov2d = T S T^T (+ dilation); Gc = [[ga, gbb/2], [gbb/2, gc]]
    const double Gc01 = 0.5 * gbb;
    const float* T = g.T;
    // Gc T (2x3)
    double GT[6];
    for (int k = 0; k < 3; ++k) {
      GT[k] = ga * T[k] + Gc01 * T[3 + k];
      GT[3 + k] = Gc01 * T[k] + gc * T[3 + k];
    }
    // dL/dT = 2 Gc T S, S symmetric with rows (S0 S1 S2), (S1 S3 S4), (S2 S4 S5)
    const double S0 = g.S[0], S1 = g.S[1], S2 = g.S[2], S3 = g.S[3], S4 = g.S[4], S5 = g.S[5];
    double dT[6];
    for (int r0 = 0; r0 < 2; ++r0) {
      const double* G = GT + 3 * r0;
      dT[3 * r0 + 0] = 2.0 * (G[0] * S0 + G[1] * S1 + G[2] * S2);
      dT[3 * r0 + 1] = 2.0 * (G[0] * S1 + G[1] * S3 + G[2] * S4);
      dT[3 * r0 + 2] = 2.0 * (G[0] * S2 + G[1] * S4 + G[2] * S5);
    }
    // T = J W with J = [[j00, 0, j02], [0, j11, j12]]
    double gj00 = 0.0, gj02 = 0.0, gj11 = 0.0, gj12 = 0.0;
    for (int k = 0; k < 3; ++k) {
      gj00 += dT[k] * cam.r[k];
      gj02 += dT[k] * cam.r[6 + k];
      gj11 += dT[3 + k] * cam.r[3 + k];
      gj12 += dT[3 + k] * cam.r[6 + k];
    }
    // j00 = fx/vz, j02 = -fx txc/vz (txc = clamp(vx/vz)), same for y
    gvz += -fx * iz2 * gj00 - fy * iz2 * gj11;
    gvz += fx * static_cast<double>(g.txc) * iz2 * gj02 + fy * static_cast<double>(g.tyc) * iz2 * gj12;
    if (g.tx >= cam.lim_x_lo && g.tx <= cam.lim_x_hi) {
      gvx += -fx * iz2 * gj02;
      gvz += fx * static_cast<double>(g.vx) * iz2 * iz * gj02;
    }
    if (g.ty >= cam.lim_y_lo && g.ty <= cam.lim_y_hi) {
      gvy += -fy * iz2 * gj12;
      gvz += fy * static_cast<double>(g.vy) * iz2 * iz * gj12;
    }
    // v = W p + t
    gm[0] = static_cast<float>(gm[0] + (cam.r[0] * gvx + cam.r[3] * gvy + cam.r[6] * gvz));
    gm[1] = static_cast<float>(gm[1] + (cam.r[1] * gvx + cam.r[4] * gvy + cam.r[7] * gvz));
    gm[2] = static_cast<float>(gm[2] + (cam.r[2] * gvx + cam.r[5] * gvy + cam.r[8] * gvz));

    // dL/dS = T^T Gc T (symmetric); S = M M^T, M = R diag(s) (the forward's float32 M):
    // dL/dM = 2 dS M; dL/dR[r][k] = dL/dM[r][k] s[k] and dL/ds[k] = sum_r dL/dM[r][k] R[r][k].
    // Each dL/dR[r][k] goes straight into the gradient of the normalised quaternion (w, x, y, z)
    // of R (nothing 3x3 is kept).
    const double w = g.qw, x = g.qx, y = g.qy, z = g.qz;
    double gw = 0.0, gx = 0.0, gy = 0.0, gz = 0.0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const double sk = g.s[k];
      double ds = 0.0;
#pragma unroll
      for (int r0 = 0; r0 < 3; ++r0) {
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const double dSrj = static_cast<double>(g.T[r0]) * GT[j] + static_cast<double>(g.T[3 + r0]) * GT[3 + j];
          acc += dSrj * static_cast<double>(g.M[3 * j + k]);
        }
        const double dMrk = 2.0 * acc;
        ds += dMrk * static_cast<double>(g.R[3 * r0 + k]);
        quat_grad_add(3 * r0 + k, dMrk * sk, w, x, y, z, gw, gx, gy, gz);
      }
      gdl[k] = static_cast<float>(ds * sk);
    }
    gw *= 2.0;
    gx *= 2.0;
    gy *= 2.0;
    gz *= 2.0;
    const double qd = w * gw + x * gx + y * gy + z * gz;
    const double qinv = g.qinv;
    gq = make_float4(static_cast<float>((gw - w * qd) * qinv), static_cast<float>((gx - x * qd) * qinv),
                     static_cast<float>((gy - y * qd) * qinv), static_cast<float>((gz - z * qd) * qinv));
  }
  if (valid) {
    g_means[3 * i] = gm[0];
    g_means[3 * i + 1] = gm[1];
    g_means[3 * i + 2] = gm[2];
    g_log_scales[3 * i] = gdl[0];
    g_log_scales[3 * i + 1] = gdl[1];
    g_log_scales[3 * i + 2] = gdl[2];
    g_quats[i] = gq;
    g_opacity[i] = gop;
  }
}

}  // namespace gs

using namespace gs;

template <int K>
static void launch_pre_fwd(int64_t blocks, hipStream_t st, const float* means, const float* ls,
                           const float* quats, const float* op, ShPtr sh, int64_t n,
                           int active, const CamK& cam, float* rec, uint32_t* touched, uint32_t* dkeys,
                           uint32_t* wave_counts) {
  hipLaunchKernelGGL(preprocess_fwd_kernel<K>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     st, means, ls, reinterpret_cast<const float4*>(quats), op, sh, n, active, cam,
                     reinterpret_cast<SplatRec*>(rec), touched, dkeys, wave_counts);
}

template <int K>
static void launch_pre_bwd(int64_t blocks, hipStream_t st, const float* means, const float* ls,
                           const float* quats, const float* op, ShPtr sh, int64_t n,
                           int active, const CamK& cam, const uint32_t* touched,
                           const float* g2, const double* c64, float* gm, float* gls, float* gq, float* gop,
                           ShOut gsh) {
  hipLaunchKernelGGL(preprocess_bwd_kernel<K>, dim3(static_cast<unsigned>(blocks)), dim3(kPreBwdWaves * 64), 0,
                     st, means, ls, reinterpret_cast<const float4*>(quats), op, sh, n, active, cam,
                     touched, g2, c64, gm, gls,
                     reinterpret_cast<float4*>(gq), gop, gsh);
}

static int check_sh(int sh_coeffs, int sh_degree) {
  GS_REQUIRE(sh_coeffs == 1 || sh_coeffs == 4 || sh_coeffs == 9 || sh_coeffs == 16, GS_ERR_ARG,
             "sh_coeffs must be 1, 4, 9 or 16 (got %d)", sh_coeffs);
  GS_REQUIRE(sh_degree >= 0 && (sh_degree + 1) * (sh_degree + 1) <= sh_coeffs, GS_ERR_ARG,
             "sh_degree %d needs more than %d coefficients", sh_degree, sh_coeffs);
  return GS_OK;
}

extern "C" int gs_preprocess_fwd(const float* means, const float* log_scales, const float* quats,
                                 const float* opacity_logits, const float* sh, const float* sh_rest,
                                 int64_t n, int sh_coeffs, int sh_degree, const gs_camera* cam,
                                 float* splat_rec, uint32_t* tiles_touched, uint32_t* depth_keys,
                                 uint32_t* wave_counts, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_ARG, "n must be >= 0");
  if (int e = check_cam(cam)) return e;
  if (int e = check_sh(sh_coeffs, sh_degree)) return e;
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && log_scales && quats && opacity_logits && sh && splat_rec && tiles_touched,
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(!(sh_rest && sh_coeffs == 1), GS_ERR_ARG, "sh_rest given for a DC-only model");
  GS_REQUIRE(aligned(quats, 16) && aligned(splat_rec, 16), GS_ERR_ALIGN,
             "quats and splat_rec must be 16-byte aligned");
  const CamK k = make_cam(*cam);
  const int active = (sh_degree + 1) * (sh_degree + 1);
  const int64_t blocks = (n + 255) / 256;
  hipStream_t st = as_stream(stream);
  const ShPtr shp{sh, sh_rest};
  switch (sh_coeffs) {
    case 1: launch_pre_fwd<1>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, splat_rec, tiles_touched, depth_keys, wave_counts); break;
    case 4: launch_pre_fwd<4>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, splat_rec, tiles_touched, depth_keys, wave_counts); break;
    case 9: launch_pre_fwd<9>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, splat_rec, tiles_touched, depth_keys, wave_counts); break;
    default: launch_pre_fwd<16>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, splat_rec, tiles_touched, depth_keys, wave_counts); break;
  }
  return check_launch("preprocess_fwd");
}

extern "C" int gs_preprocess_bwd(const float* means, const float* log_scales, const float* quats,
                                 const float* opacity_logits, const float* sh, const float* sh_rest,
                                 int64_t n, int sh_coeffs, int sh_degree, const gs_camera* cam,
                                 const uint32_t* tiles_touched,
                                 const float* grad2d, const double* grad_conic64, float* grad_means,
                                 float* grad_log_scales,
                                 float* grad_quats, float* grad_opacity_logits, float* grad_sh,
                                 float* grad_sh_rest, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_ARG, "n must be >= 0");
  if (int e = check_cam(cam)) return e;
  if (int e = check_sh(sh_coeffs, sh_degree)) return e;
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && log_scales && quats && opacity_logits && sh && tiles_touched &&
                 grad2d && grad_means && grad_log_scales && grad_quats && grad_opacity_logits &&
                 grad_sh,
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(!sh_rest == !grad_sh_rest, GS_ERR_ARG, "sh_rest and grad_sh_rest go together");
  GS_REQUIRE(aligned(grad_conic64, 8), GS_ERR_ALIGN, "grad_conic64 must be 8-byte aligned");
  GS_REQUIRE(!(sh_rest && sh_coeffs == 1), GS_ERR_ARG, "sh_rest given for a DC-only model");
  GS_REQUIRE(aligned(quats, 16) && aligned(grad_quats, 16), GS_ERR_ALIGN,
             "quats and grad_quats must be 16-byte aligned");
  const CamK k = make_cam(*cam);
  const int active = (sh_degree + 1) * (sh_degree + 1);
  const int64_t blocks = (n + kPreBwdWaves * 64 - 1) / (kPreBwdWaves * 64);
  hipStream_t st = as_stream(stream);
  const ShPtr shp{sh, sh_rest};
  const ShOut gsh{grad_sh, grad_sh_rest};
  switch (sh_coeffs) {
    case 1: launch_pre_bwd<1>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, tiles_touched, grad2d, grad_conic64, grad_means, grad_log_scales, grad_quats, grad_opacity_logits, gsh); break;
    case 4: launch_pre_bwd<4>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, tiles_touched, grad2d, grad_conic64, grad_means, grad_log_scales, grad_quats, grad_opacity_logits, gsh); break;
    case 9: launch_pre_bwd<9>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, tiles_touched, grad2d, grad_conic64, grad_means, grad_log_scales, grad_quats, grad_opacity_logits, gsh); break;
    default: launch_pre_bwd<16>(blocks, st, means, log_scales, quats, opacity_logits, shp, n, active, k, tiles_touched, grad2d, grad_conic64, grad_means, grad_log_scales, grad_quats, grad_opacity_logits, gsh); break;
  }
  return check_launch("preprocess_bwd");
}

// ---------------------------------------------------------------------------------------
// Densification statistics
// ---------------------------------------------------------------------------------------
namespace gs {

__global__ void densification_stats_kernel(const float* __restrict__ grad2d, const uint32_t* __restrict__ touched,
                                           int64_t n, float sx, float sy, int rows, float* __restrict__ info) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n || touched[i] == 0u) return;
  const float* g = grad2d + i * kGrad2D;
  const float gx = g[0] * sx, gy = g[1] * sy;
  info[i] += 1.0f;
  info[n + i] += sqrtf(fmaf(gx, gx, gy * gy));
  if (rows > 2) {
    const float ax = g[9] * sx, ay = g[10] * sy;
    info[2 * n + i] += sqrtf(fmaf(ax, ax, ay * ay));
  }
}

}  // namespace gs

extern "C" int gs_densification_stats(const float* grad2d, const uint32_t* tiles_touched, int64_t n, int width,
                                      int height, int rows, float* info, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && width > 0 && height > 0 && (rows == 2 || rows == 3), GS_ERR_ARG,
             "invalid densification_stats arguments");
  if (n == 0) return GS_OK;
  GS_REQUIRE(grad2d && tiles_touched && info, GS_ERR_ARG, "null pointer argument");
  hipLaunchKernelGGL(densification_stats_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     as_stream(stream), grad2d, tiles_touched, n, 0.5f * static_cast<float>(width),
                     0.5f * static_cast<float>(height), rows, info);
  return check_launch("densification_stats");
}
