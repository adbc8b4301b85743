// Fused Adam for the Gaussian parameters: every parameter group in one launch, each thread
// four consecutive elements (16-byte accesses when the group allows), an optional per-primitive
// visibility mask (invisible rows are neither read nor written) and optional bfloat16 moments
// written with stochastic rounding. The update rule is the one of
// cluster/patches/fastergs_lean_adam.patch:96-139 (same rounding steps, so float32 results are
// bit-identical to it); it is HBM-bound: 28 bytes per element with float32 moments.
#include "gs_host.h"

namespace gs {

constexpr int kAdamThreads = 256;
constexpr int kAdamPerThread = 4;
constexpr int64_t kAdamBlockElems = kAdamThreads * kAdamPerThread;

struct AdamGroupK {
  const float* grad;
  float* param;
  void* m;
  void* v;
  int64_t n;        // elements
  int64_t block0;   // first block of the group
  uint32_t feat;    // elements per primitive
  uint32_t seed;
  int lowp;
  float step_size, beta1, beta2, eps, bc2;
};

struct AdamArgs {
  AdamGroupK g[GS_ADAM_MAX_GROUPS];
  int n_groups;
  const int32_t* vis;
};

// Integer hash of the stochastic rounding (the 32-bit "lowbias32" finaliser: xor-shift,
// multiply, xor-shift, multiply, xor-shift).
__device__ __forceinline__ uint32_t sr_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ uint16_t to_bf16_sr(float f, uint32_t rnd) {
  return static_cast<uint16_t>((__float_as_uint(f) + (rnd & 0xffffu)) >> 16);
}

__device__ __forceinline__ void adam_elem(const AdamGroupK& G, float g, float& p, float& m, float& v) {
  const float gsq = g * g;
  m = fmaf(G.beta1, m - g, g);
  v = fmaf(G.beta2, v - gsq, gsq);
  const float denom = sqrtf(v) * G.bc2 + G.eps;
  p = p - (G.step_size * m) / denom;
}

__global__ __launch_bounds__(kAdamThreads) void adam_kernel(AdamArgs a) {
  int gi = 0;
#pragma unroll
  for (int k = 1; k < GS_ADAM_MAX_GROUPS; ++k)
    if (k < a.n_groups && static_cast<int64_t>(blockIdx.x) >= a.g[k].block0) gi = k;
  const AdamGroupK& G = a.g[gi];
  const int64_t e0 = (static_cast<int64_t>(blockIdx.x) - G.block0) * kAdamBlockElems +
                     static_cast<int64_t>(threadIdx.x) * kAdamPerThread;
  if (e0 >= G.n) return;
  const int cnt = static_cast<int>(min<int64_t>(kAdamPerThread, G.n - e0));
  bool live[kAdamPerThread];
  bool any = false;
  int64_t row0 = 0;
  uint32_t rem = 0;
  if (a.vis) {  // row of element e0 + k = row0 + (rem + k) / feat
    if (G.n <= 0xffffffffLL) {
      const uint32_t e = static_cast<uint32_t>(e0);
      const uint32_t r = e / G.feat;
      row0 = r;
      rem = e - r * G.feat;
    } else {
      row0 = e0 / G.feat;
      rem = static_cast<uint32_t>(e0 - row0 * G.feat);
    }
  }
#pragma unroll
  for (int k = 0; k < kAdamPerThread; ++k) {
    live[k] = k < cnt && (a.vis == nullptr || a.vis[row0 + (rem + k) / G.feat] != 0);
    any = any || live[k];
  }
  if (!any) return;
  // 16-byte accesses whenever the four elements exist and are aligned; elements of hidden rows
  // are written back bit-identical (no other thread owns them)
  const bool al = cnt == kAdamPerThread &&
                  ((reinterpret_cast<uintptr_t>(G.grad + e0) | reinterpret_cast<uintptr_t>(G.param + e0)) & 15u) == 0;
  if (al) {
    float g[kAdamPerThread], p[kAdamPerThread], m[kAdamPerThread], v[kAdamPerThread];
    const float4 g4 = *reinterpret_cast<const float4*>(G.grad + e0);
    const float4 p4 = *reinterpret_cast<const float4*>(G.param + e0);
    g[0] = g4.x; g[1] = g4.y; g[2] = g4.z; g[3] = g4.w;
    p[0] = p4.x; p[1] = p4.y; p[2] = p4.z; p[3] = p4.w;
    if (!G.lowp && ((reinterpret_cast<uintptr_t>(static_cast<float*>(G.m) + e0) |
                     reinterpret_cast<uintptr_t>(static_cast<float*>(G.v) + e0)) & 15u) == 0) {
      const float4 m4 = *reinterpret_cast<const float4*>(static_cast<float*>(G.m) + e0);
      const float4 v4 = *reinterpret_cast<const float4*>(static_cast<float*>(G.v) + e0);
      m[0] = m4.x; m[1] = m4.y; m[2] = m4.z; m[3] = m4.w;
      v[0] = v4.x; v[1] = v4.y; v[2] = v4.z; v[3] = v4.w;
#pragma unroll
      for (int k = 0; k < kAdamPerThread; ++k)
        if (live[k]) adam_elem(G, g[k], p[k], m[k], v[k]);
      *reinterpret_cast<float4*>(G.param + e0) = make_float4(p[0], p[1], p[2], p[3]);
      *reinterpret_cast<float4*>(static_cast<float*>(G.m) + e0) = make_float4(m[0], m[1], m[2], m[3]);
      *reinterpret_cast<float4*>(static_cast<float*>(G.v) + e0) = make_float4(v[0], v[1], v[2], v[3]);
      return;
    }
    if (G.lowp && ((reinterpret_cast<uintptr_t>(static_cast<uint16_t*>(G.m) + e0) |
                    reinterpret_cast<uintptr_t>(static_cast<uint16_t*>(G.v) + e0)) & 7u) == 0) {
      const uint2 mb = *reinterpret_cast<const uint2*>(static_cast<uint16_t*>(G.m) + e0);
      const uint2 vb = *reinterpret_cast<const uint2*>(static_cast<uint16_t*>(G.v) + e0);
      uint32_t mw[2] = {mb.x, mb.y}, vw[2] = {vb.x, vb.y};
#pragma unroll
      for (int k = 0; k < kAdamPerThread; ++k) {
        const uint32_t sh = 16u * (k & 1);
        m[k] = __uint_as_float(((mw[k >> 1] >> sh) & 0xffffu) << 16);
        v[k] = __uint_as_float(((vw[k >> 1] >> sh) & 0xffffu) << 16);
        if (!live[k]) continue;
        adam_elem(G, g[k], p[k], m[k], v[k]);
        const int64_t idx = e0 + k;
        const uint32_t r1 = sr_hash(static_cast<uint32_t>(idx) ^ G.seed);
        const uint32_t r2 = sr_hash(r1);
        const uint32_t keep = 0xffffu << (16u - sh);  // the other half-word
        mw[k >> 1] = (mw[k >> 1] & keep) | (static_cast<uint32_t>(to_bf16_sr(m[k], r1)) << sh);
        vw[k >> 1] = (vw[k >> 1] & keep) | (static_cast<uint32_t>(to_bf16_sr(v[k], r2)) << sh);
      }
      *reinterpret_cast<float4*>(G.param + e0) = make_float4(p[0], p[1], p[2], p[3]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(G.m) + e0) = make_uint2(mw[0], mw[1]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(G.v) + e0) = make_uint2(vw[0], vw[1]);
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < kAdamPerThread; ++k) {
    if (!live[k]) continue;
    const int64_t idx = e0 + k;
    float pk = G.param[idx], mk, vk;
    if (G.lowp) {
      mk = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(G.m)[idx]) << 16);
      vk = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(G.v)[idx]) << 16);
    } else {
      mk = static_cast<const float*>(G.m)[idx];
      vk = static_cast<const float*>(G.v)[idx];
    }
    adam_elem(G, G.grad[idx], pk, mk, vk);
    G.param[idx] = pk;
    if (G.lowp) {
      const uint32_t r1 = sr_hash(static_cast<uint32_t>(idx) ^ G.seed);
      const uint32_t r2 = sr_hash(r1);
      static_cast<uint16_t*>(G.m)[idx] = to_bf16_sr(mk, r1);
      static_cast<uint16_t*>(G.v)[idx] = to_bf16_sr(vk, r2);
    } else {
      static_cast<float*>(G.m)[idx] = mk;
      static_cast<float*>(G.v)[idx] = vk;
    }
  }
}

}  // namespace gs

using namespace gs;

extern "C" int gs_adam_step(const gs_adam_group* groups, int n_groups, int64_t n_primitives,
                            const int32_t* visibility, void* stream) {
  clear_error();
  GS_REQUIRE(groups && n_groups >= 1 && n_groups <= GS_ADAM_MAX_GROUPS, GS_ERR_ARG,
             "need 1 to %d parameter groups", GS_ADAM_MAX_GROUPS);
  GS_REQUIRE(n_primitives >= 0, GS_ERR_ARG, "n_primitives must be >= 0");
  AdamArgs a = {};
  a.n_groups = n_groups;
  a.vis = visibility;
  int64_t blocks = 0;
  for (int i = 0; i < n_groups; ++i) {
    const gs_adam_group& q = groups[i];
    GS_REQUIRE(q.n_elements >= 0, GS_ERR_ARG, "group %d: n_elements must be >= 0", i);
    GS_REQUIRE(q.n_elements == 0 || (q.grad && q.param && q.exp_avg && q.exp_avg_sq), GS_ERR_ARG,
               "group %d: null pointer", i);
    GS_REQUIRE(q.moment_dtype == GS_FLOAT32 || q.moment_dtype == GS_BFLOAT16, GS_ERR_ARG,
               "group %d: moments must be GS_FLOAT32 or GS_BFLOAT16", i);
    GS_REQUIRE(q.step >= 1, GS_ERR_ARG, "group %d: step must be >= 1", i);
    GS_REQUIRE(n_primitives > 0 ? q.n_elements % n_primitives == 0 : q.n_elements == 0, GS_ERR_ARG,
               "group %d: %lld elements are not rows of %lld primitives", i,
               static_cast<long long>(q.n_elements), static_cast<long long>(n_primitives));
    const int64_t feat = n_primitives > 0 ? q.n_elements / n_primitives : 1;
    GS_REQUIRE(feat <= 0xffffffffLL, GS_ERR_ARG, "group %d: too many elements per primitive", i);
    AdamGroupK& g = a.g[i];
    g.grad = q.grad;
    g.param = q.param;
    g.m = q.exp_avg;
    g.v = q.exp_avg_sq;
    g.n = q.n_elements;
    g.block0 = blocks;
    g.feat = static_cast<uint32_t>(feat > 0 ? feat : 1);
    g.lowp = q.moment_dtype == GS_BFLOAT16;
    g.seed = 0x9E3779B9u * static_cast<uint32_t>(q.step) + 0x85EBCA6Bu;
    const double bc1 = 1.0 / (1.0 - pow(q.beta1, q.step));
    const double bc2 = 1.0 / sqrt(1.0 - pow(q.beta2, q.step));
    g.step_size = static_cast<float>(q.lr * bc1);
    g.beta1 = static_cast<float>(q.beta1);
    g.beta2 = static_cast<float>(q.beta2);
    g.eps = static_cast<float>(q.eps);
    g.bc2 = static_cast<float>(bc2);
    blocks += (q.n_elements + kAdamBlockElems - 1) / kAdamBlockElems;
  }
  for (int i = n_groups; i < GS_ADAM_MAX_GROUPS; ++i) a.g[i].block0 = INT64_MAX;
  if (blocks == 0) return GS_OK;
  GS_REQUIRE(blocks < (int64_t(1) << 31), GS_ERR_ARG, "too many elements");
  hipLaunchKernelGGL(adam_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kAdamThreads), 0, as_stream(stream), a);
  return check_launch("adam_step");
}
