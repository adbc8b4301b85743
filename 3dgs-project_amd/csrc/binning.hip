// Tile binning: exclusive scan, instance (key, value) emission, stable LSD radix sort of the
// 64-bit keys (tile << 32 | orderable depth), per-tile ranges and 32-entry buckets.
//
// The radix sort is reduce-then-scan per 8-bit digit: a histogram kernel, a device-wide
// exclusive scan of the digit-major histogram table, and a scatter kernel that ranks keys
// stably inside its block (wavefront match over the 8 digit bits with ballots, then a
// per-digit prefix over the block's four wavefronts). No kernel waits on another
// workgroup, so there is no forward-progress requirement.
#include "gs_host.h"

namespace gs {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;  // 2048 values per workgroup

constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;
constexpr int kSortTile = kSortThreads * kSortRounds;  // 4096 keys per workgroup

__device__ __forceinline__ uint64_t lanemask_lt(int lane) {
  return (lane == 0) ? 0ull : (~0ull >> (64 - lane));
}

// Inclusive scan of one value per thread across a 256-thread workgroup; returns the
// workgroup total through `total`.
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t v, uint32_t* s_wave,
                                                         uint32_t& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  if (lane == 63) s_wave[wave] = v;
  __syncthreads();
  uint32_t before = 0;
  for (int w = 0; w < wave; ++w) before += s_wave[w];
  total = s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
  __syncthreads();
  return v + before;
}

// Exclusive scan of one 2048-value tile. `block_sums` (if not null) receives the tile total;
// otherwise out[n] receives it.
__global__ __launch_bounds__(kScanThreads) void scan_tile_kernel(const uint32_t* __restrict__ in,
                                                                 uint32_t* __restrict__ out,
                                                                 int64_t n,
                                                                 uint32_t* __restrict__ block_sums) {
  __shared__ uint32_t s_v[kScanTile];
  __shared__ uint32_t s_wave[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int k = threadIdx.x; k < kScanTile; k += kScanThreads) {
    const int64_t idx = base + k;
    s_v[k] = idx < n ? in[idx] : 0u;
  }
  __syncthreads();
  uint32_t local[kScanItems];
  uint32_t sum = 0;
#pragma unroll
  for (int e = 0; e < kScanItems; ++e) {
    local[e] = s_v[threadIdx.x * kScanItems + e];
    sum += local[e];
  }
  uint32_t total;
  const uint32_t incl = block_inclusive_scan(sum, s_wave, total);
  uint32_t run = incl - sum;
#pragma unroll
  for (int e = 0; e < kScanItems; ++e) {
    s_v[threadIdx.x * kScanItems + e] = run;
    run += local[e];
  }
  __syncthreads();
  for (int k = threadIdx.x; k < kScanTile; k += kScanThreads) {
    const int64_t idx = base + k;
    if (idx < n) out[idx] = s_v[k];
  }
  if (threadIdx.x == 0) {
    if (block_sums) {
      block_sums[blockIdx.x] = total;
    } else {
      out[n] = total;
    }
  }
}

__global__ __launch_bounds__(kScanThreads) void scan_add_kernel(uint32_t* __restrict__ out,
                                                                int64_t n,
                                                                const uint32_t* __restrict__ offs,
                                                                int64_t n_blocks) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  const uint32_t add = offs[blockIdx.x];
  for (int k = threadIdx.x; k < kScanTile; k += kScanThreads) {
    const int64_t idx = base + k;
    if (idx < n) out[idx] += add;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = offs[n_blocks];
}

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static size_t scan_ws(int64_t n) {
  if (n <= kScanTile) return 0;
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  return align_up(nb * 4) + align_up((nb + 1) * 4) + scan_ws(nb);
}

static void scan_rec(const uint32_t* in, uint32_t* out, int64_t n, char* ws, hipStream_t st) {
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  if (nb <= 1) {
    hipLaunchKernelGGL(scan_tile_kernel, dim3(1), dim3(kScanThreads), 0, st, in, out, n, nullptr);
    return;
  }
  uint32_t* sums = reinterpret_cast<uint32_t*>(ws);
  uint32_t* sums_scan = reinterpret_cast<uint32_t*>(ws + align_up(nb * 4));
  char* next = ws + align_up(nb * 4) + align_up((nb + 1) * 4);
  hipLaunchKernelGGL(scan_tile_kernel, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, st,
                     in, out, n, sums);
  scan_rec(sums, sums_scan, nb, next, st);
  hipLaunchKernelGGL(scan_add_kernel, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, st,
                     out, n, sums_scan, nb);
}

// ---------------------------------------------------------------------------------------
// Instances
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void emit_instances_kernel(
    const SplatRec* __restrict__ rec, const uint32_t* __restrict__ touched,
    const uint32_t* __restrict__ offsets, int64_t n, int tiles_x, uint64_t* __restrict__ keys,
    uint32_t* __restrict__ vals) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n || touched[i] == 0u) return;
  const SplatRec r = rec[i];
  const uint64_t dkey = float_order_key(r.b.z);
  const uint32_t off = offsets[i];
  for_each_touched_tile(r.a, r.b, r.d, tiles_x, [&](int tile, int k) {
    keys[off + k] = (static_cast<uint64_t>(tile) << 32) | dkey;
    vals[off + k] = static_cast<uint32_t>(i);
  });
}

// ---------------------------------------------------------------------------------------
// Radix sort
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint64_t* __restrict__ keys,
                                                                  int64_t m, int shift,
                                                                  uint32_t* __restrict__ hist,
                                                                  int n_blocks) {
  __shared__ uint32_t s_h[256];
  s_h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
#pragma unroll 4
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t idx = base + r * kSortThreads + threadIdx.x;
    if (idx < m) {
      const uint32_t d = static_cast<uint32_t>(keys[idx] >> shift) & 255u;
      atomicAdd(&s_h[d], 1u);
    }
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * n_blocks + blockIdx.x] = s_h[threadIdx.x];
}

__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint64_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint64_t* __restrict__ kout, uint32_t* __restrict__ vout, int64_t m, int shift,
    const uint32_t* __restrict__ offs, int n_blocks) {
  __shared__ uint32_t s_base[256];
  __shared__ uint32_t s_cnt[4][256];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  s_base[tid] = offs[static_cast<int64_t>(tid) * n_blocks + blockIdx.x];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
  const uint64_t lt = lanemask_lt(lane);
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t idx = base + r * kSortThreads + tid;
    const bool valid = idx < m;
    uint64_t key = 0;
    uint32_t val = 0;
    uint32_t d = 0;
    if (valid) {
      key = kin[idx];
      val = vin[idx];
      d = static_cast<uint32_t>(key >> shift) & 255u;
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) s_cnt[w][tid] = 0;
    uint64_t peers = __ballot(valid ? 1 : 0);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool set = (d >> bit) & 1u;
      const uint64_t bm = __ballot(set ? 1 : 0);
      peers &= set ? bm : ~bm;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lt));
    const uint32_t cnt = static_cast<uint32_t>(__popcll(peers));
    __syncthreads();  // s_cnt cleared, s_base final from the previous round
    if (valid && rank == 0) s_cnt[wave][d] = cnt;
    __syncthreads();
    {
      const uint32_t c0 = s_cnt[0][tid], c1 = s_cnt[1][tid], c2 = s_cnt[2][tid], c3 = s_cnt[3][tid];
      const uint32_t run = s_base[tid];
      s_cnt[0][tid] = run;
      s_cnt[1][tid] = run + c0;
      s_cnt[2][tid] = run + c0 + c1;
      s_cnt[3][tid] = run + c0 + c1 + c2;
      s_base[tid] = run + c0 + c1 + c2 + c3;
    }
    __syncthreads();
    if (valid) {
      const uint32_t pos = s_cnt[wave][d] + rank;
      kout[pos] = key;
      vout[pos] = val;
    }
    __syncthreads();  // s_cnt is cleared at the top of the next round
  }
}

// ---------------------------------------------------------------------------------------
// Ranges and buckets
// ---------------------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void fill_f32_kernel(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void ranges_kernel(const uint64_t* __restrict__ keys, int64_t m,
                              uint32_t* __restrict__ ranges) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= m) return;
  const uint32_t t = static_cast<uint32_t>(keys[p] >> 32);
  if (p == 0 || static_cast<uint32_t>(keys[p - 1] >> 32) != t) ranges[2 * t] = static_cast<uint32_t>(p);
  if (p == m - 1 || static_cast<uint32_t>(keys[p + 1] >> 32) != t)
    ranges[2 * t + 1] = static_cast<uint32_t>(p + 1);
}

__global__ void bucket_count_kernel(const uint32_t* __restrict__ ranges, int n_tiles,
                                    uint32_t* __restrict__ counts) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tiles) return;
  const uint32_t len = ranges[2 * t + 1] - ranges[2 * t];
  counts[t] = (len + kBucket - 1) / kBucket;
}

// One thread per bucket slot: binary search of the tile whose bucket range holds b.
__global__ void bucket_fill_kernel(const uint32_t* __restrict__ boff, int n_tiles,
                                   uint32_t* __restrict__ b2t, int64_t n_max) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= n_max) return;
  if (b >= static_cast<int64_t>(boff[n_tiles])) {
    b2t[b] = 0xffffffffu;
    return;
  }
  int lo = 0, hi = n_tiles - 1;  // largest t with boff[t] <= b
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (static_cast<int64_t>(boff[mid]) <= b) lo = mid;
    else hi = mid - 1;
  }
  b2t[b] = static_cast<uint32_t>(lo);
}

}  // namespace gs

using namespace gs;

static inline unsigned grid_for(int64_t n, int threads) {
  return static_cast<unsigned>((n + threads - 1) / threads);
}

extern "C" size_t gs_scan_workspace_size(int64_t n) { return scan_ws(n < 0 ? 0 : n); }

extern "C" int gs_scan_u32(const uint32_t* in, uint32_t* out, int64_t n, void* workspace,
                           size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && out != nullptr && (n == 0 || in != nullptr), GS_ERR_ARG,
             "invalid scan arguments");
  GS_REQUIRE(workspace_bytes >= scan_ws(n) && (scan_ws(n) == 0 || workspace), GS_ERR_WORKSPACE,
             "scan workspace too small: need %zu bytes", scan_ws(n));
  hipStream_t st = as_stream(stream);
  if (n == 0) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, st, out, int64_t(1), 0u);
    return check_launch("scan");
  }
  scan_rec(in, out, n, static_cast<char*>(workspace), st);
  return check_launch("scan");
}

static int tile_bits(int n_tiles) {
  int b = 0;
  while ((1 << b) < n_tiles) ++b;
  return b;
}

static int sort_passes(int n_tiles) { return (32 + tile_bits(n_tiles) + 7) / 8; }

extern "C" size_t gs_bin_workspace_size(int64_t m, int n_tiles) {
  if (m < 0 || n_tiles <= 0) return 0;
  const int64_t nb = (m + kSortTile - 1) / kSortTile;
  const int64_t hist = 256 * (nb > 0 ? nb : 1);
  size_t s = align_up(m * 8) + align_up(m * 4);  // ping-pong keys and values
  s += align_up(hist * 4) + align_up((hist + 1) * 4) + scan_ws(hist);
  s += align_up(static_cast<size_t>(n_tiles) * 4) + scan_ws(n_tiles);
  return s;
}

extern "C" int gs_bin_fill_3d(const float* splat_rec, const uint32_t* tiles_touched,
                              const uint32_t* offsets, int64_t n, const gs_camera* cam, int64_t m,
                              uint64_t* sorted_keys, uint32_t* point_list, uint32_t* ranges,
                              uint32_t* bucket_offsets, void* workspace, size_t workspace_bytes,
                              void* stream) {
  clear_error();
  if (int e = check_cam(cam)) return e;
  GS_REQUIRE(n >= 0 && m >= 0 && m < (int64_t(1) << 32), GS_ERR_ARG, "invalid sizes n=%lld m=%lld",
             static_cast<long long>(n), static_cast<long long>(m));
  GS_REQUIRE(ranges && bucket_offsets, GS_ERR_ARG, "null output");
  const CamK k = make_cam(*cam);
  const int n_tiles = k.tiles_x * k.tiles_y;
  const size_t need = gs_bin_workspace_size(m, n_tiles);
  GS_REQUIRE(workspace_bytes >= need && workspace, GS_ERR_WORKSPACE,
             "binning workspace too small: need %zu bytes", need);
  GS_REQUIRE(m == 0 || (splat_rec && tiles_touched && offsets && sorted_keys && point_list),
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16), GS_ERR_ALIGN, "splat_rec must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  uint64_t* k_alt = reinterpret_cast<uint64_t*>(ws);
  ws += align_up(m * 8);
  uint32_t* v_alt = reinterpret_cast<uint32_t*>(ws);
  ws += align_up(m * 4);
  const int64_t nb = (m + kSortTile - 1) / kSortTile;
  const int64_t hist_n = 256 * (nb > 0 ? nb : 1);
  uint32_t* hist = reinterpret_cast<uint32_t*>(ws);
  ws += align_up(hist_n * 4);
  uint32_t* hist_scan = reinterpret_cast<uint32_t*>(ws);
  ws += align_up((hist_n + 1) * 4);
  char* hist_ws = ws;
  ws += scan_ws(hist_n);
  uint32_t* bcount = reinterpret_cast<uint32_t*>(ws);
  ws += align_up(static_cast<size_t>(n_tiles) * 4);
  char* tile_ws = ws;

  hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(2 * int64_t(n_tiles), 256)), dim3(256), 0, st,
                     ranges, 2 * int64_t(n_tiles), 0u);
  if (m > 0) {
    const int passes = sort_passes(n_tiles);
    // emit into the buffer that ends up holding the result after `passes` ping-pongs
    uint64_t* k0 = (passes % 2 == 0) ? sorted_keys : k_alt;
    uint32_t* v0 = (passes % 2 == 0) ? point_list : v_alt;
    uint64_t* k1 = (passes % 2 == 0) ? k_alt : sorted_keys;
    uint32_t* v1 = (passes % 2 == 0) ? v_alt : point_list;
    hipLaunchKernelGGL(emit_instances_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st,
                       reinterpret_cast<const SplatRec*>(splat_rec), tiles_touched, offsets, n,
                       k.tiles_x, k0, v0);
    for (int p = 0; p < passes; ++p) {
      const int shift = 8 * p;
      hipLaunchKernelGGL(radix_hist_kernel, dim3(static_cast<unsigned>(nb)), dim3(kSortThreads), 0,
                         st, k0, m, shift, hist, static_cast<int>(nb));
      scan_rec(hist, hist_scan, hist_n, hist_ws, st);
      hipLaunchKernelGGL(radix_scatter_kernel, dim3(static_cast<unsigned>(nb)), dim3(kSortThreads),
                         0, st, k0, v0, k1, v1, m, shift, hist_scan, static_cast<int>(nb));
      std::swap(k0, k1);
      std::swap(v0, v1);
    }
    hipLaunchKernelGGL(ranges_kernel, dim3(grid_for(m, 256)), dim3(256), 0, st, sorted_keys, m,
                       ranges);
  }
  hipLaunchKernelGGL(bucket_count_kernel, dim3(grid_for(n_tiles, 256)), dim3(256), 0, st, ranges,
                     n_tiles, bcount);
  scan_rec(bcount, bucket_offsets, n_tiles, tile_ws, st);
  return check_launch("bin_fill_3d");
}

extern "C" int gs_bucket_fill(const uint32_t* bucket_offsets, int n_tiles, uint32_t* bucket_to_tile,
                              int64_t n_buckets_max, void* stream) {
  clear_error();
  GS_REQUIRE(n_tiles > 0 && n_buckets_max >= 0 && bucket_offsets, GS_ERR_ARG,
             "invalid bucket_fill arguments");
  GS_REQUIRE(n_buckets_max == 0 || bucket_to_tile, GS_ERR_ARG, "null bucket_to_tile");
  if (n_buckets_max == 0) return GS_OK;
  hipLaunchKernelGGL(bucket_fill_kernel, dim3(grid_for(n_buckets_max, 256)), dim3(256), 0,
                     as_stream(stream), bucket_offsets, n_tiles, bucket_to_tile, n_buckets_max);
  return check_launch("bucket_fill");
}

// zero-fill helper for the other translation units
namespace gs {
void fill_zero_f32(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, p, n, 0.0f);
}
}  // namespace gs
