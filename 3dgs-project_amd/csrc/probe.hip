// Measurement probes: the achievable HBM bandwidth (a plain copy and a read-only sweep) and
// FP32 VALU rate (independent FMA chains) of the GPU the library runs on, the ceilings the
// roofline fractions are also quoted against. The reference measured its bandwidth ceilings
// the same way (copy and read-only kernels, results/phase1/README.md:10-16).
#include "gs_host.h"

namespace gs {

constexpr int kProbeThreads = 256;
constexpr int kProbeVec = 4;  // float4 accesses per thread, all loads issued before the stores

// out[i] = in[i]: each thread copies kProbeVec float4 of one contiguous 4 KiB block per
// workgroup (the loads of a wavefront are 1 KiB runs), issuing its loads before its stores.
__global__ __launch_bounds__(kProbeThreads) void probe_copy_kernel(const float4* __restrict__ in,
                                                                   float4* __restrict__ out, int64_t n4) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kProbeThreads * kProbeVec + threadIdx.x;
  float4 v[kProbeVec];
#pragma unroll
  for (int u = 0; u < kProbeVec; ++u) {
    const int64_t i = base + u * kProbeThreads;
    if (i < n4) v[u] = in[i];
  }
#pragma unroll
  for (int u = 0; u < kProbeVec; ++u) {
    const int64_t i = base + u * kProbeThreads;
    if (i < n4) out[i] = v[u];
  }
}

// Reads every float once (kProbeVec float4 per thread, loads issued together); each wavefront
// writes one sum, so nothing is optimised away and the writes are 1/4096 of the traffic.
__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const float4* __restrict__ in, int64_t n4,
                                                                   float* __restrict__ sums) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kProbeThreads * kProbeVec + threadIdx.x;
  float4 v[kProbeVec];
#pragma unroll
  for (int u = 0; u < kProbeVec; ++u) {
    const int64_t i = base + u * kProbeThreads;
    v[u] = i < n4 ? in[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < kProbeVec; ++u) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) sums[static_cast<int64_t>(blockIdx.x) * (kProbeThreads / 64) + (threadIdx.x >> 6)] = s;
}

// 16 independent FMA chains of `iters` x 4 steps per thread (64 iters wave64 v_fma_f32 per
// wavefront, plus a few instructions of set-up and loop control), one float written per thread.
// The library is built without packed FP32, so this is the FP32 VALU ceiling its kernels face.
constexpr int kFmaChains = 16;

__global__ __launch_bounds__(kProbeThreads) void probe_fma_kernel(float* __restrict__ out, int iters, float a,
                                                                  float b) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  float x[kFmaChains];
#pragma unroll
  for (int c = 0; c < kFmaChains; ++c) x[c] = static_cast<float>(threadIdx.x) * 1e-7f + 1e-3f * c;
  for (int k = 0; k < iters; ++k) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < kFmaChains; ++c) x[c] = fmaf(x[c], a, b);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kFmaChains; ++c) s += x[c];
  out[tid] = s;
}

}  // namespace gs

using namespace gs;

static int64_t probe_blocks(int64_t n4) {
  const int64_t per_block = static_cast<int64_t>(kProbeThreads) * kProbeVec;
  return (n4 + per_block - 1) / per_block;
}

extern "C" int gs_probe_copy(const float* in, float* out, int64_t n, void* stream) {
  clear_error();
  GS_REQUIRE(in && out && n > 0 && n % 4 == 0, GS_ERR_ARG, "probe_copy: need n > 0, a multiple of 4");
  GS_REQUIRE(aligned(in, 16) && aligned(out, 16), GS_ERR_ALIGN, "probe_copy: 16-byte aligned buffers");
  const int64_t n4 = n / 4;
  GS_REQUIRE(probe_blocks(n4) <= 0x7fffffff, GS_ERR_ARG, "probe_copy: n too large");
  hipLaunchKernelGGL(probe_copy_kernel, dim3(static_cast<unsigned>(probe_blocks(n4))), dim3(kProbeThreads), 0,
                     as_stream(stream),
                     reinterpret_cast<const float4*>(in), reinterpret_cast<float4*>(out), n4);
  return check_launch("probe_copy");
}

extern "C" int64_t gs_probe_read_sums(int64_t n) { return n > 0 ? probe_blocks(n / 4) * (kProbeThreads / 64) : 0; }

extern "C" int gs_probe_read(const float* in, int64_t n, float* sums, void* stream) {
  clear_error();
  GS_REQUIRE(in && sums && n > 0 && n % 4 == 0, GS_ERR_ARG, "probe_read: need n > 0, a multiple of 4");
  GS_REQUIRE(aligned(in, 16), GS_ERR_ALIGN, "probe_read: 16-byte aligned input");
  const int64_t n4 = n / 4;
  GS_REQUIRE(probe_blocks(n4) <= 0x7fffffff, GS_ERR_ARG, "probe_read: n too large");
  hipLaunchKernelGGL(probe_read_kernel, dim3(static_cast<unsigned>(probe_blocks(n4))), dim3(kProbeThreads), 0,
                     as_stream(stream),
                     reinterpret_cast<const float4*>(in), n4, sums);
  return check_launch("probe_read");
}

extern "C" int gs_probe_fma(float* out, int64_t threads, int iters, void* stream) {
  clear_error();
  GS_REQUIRE(out && threads > 0 && threads % kProbeThreads == 0 && iters > 0, GS_ERR_ARG,
             "probe_fma: need threads > 0, a multiple of %d, and iters > 0", kProbeThreads);
  GS_REQUIRE(threads / kProbeThreads <= 0x7fffffff, GS_ERR_ARG, "probe_fma: too many threads");
  hipLaunchKernelGGL(probe_fma_kernel, dim3(static_cast<unsigned>(threads / kProbeThreads)), dim3(kProbeThreads), 0,
                     as_stream(stream), out, iters, 0.999f, 1e-3f);
  return check_launch("probe_fma");
}
