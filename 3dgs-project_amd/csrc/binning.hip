// Tile binning: exclusive scan, per-tile instance lists in (tile, depth, Gaussian index)
// order, per-tile ranges and 32-entry buckets.
//
// The order is that of a stable sort of 64-bit keys (tile << 32 | orderable depth) over
// instances emitted in Gaussian-index order, obtained in two levels: a stable 32-bit sort of
// the Gaussians by depth (N keys), emission of the instances in that order, and a stable sort
// of the instances by tile (M keys, ceil(log2 T) bits). Each sort is LSD radix with 8-bit
// digits, reduce-then-scan per digit: a histogram kernel, a device-wide exclusive scan of the
// digit-major histogram table, and a scatter kernel that ranks keys stably inside its
// workgroup. No kernel waits on another workgroup, so there is no forward-progress
// requirement.
#include "gs_host.h"

namespace gs {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;  // 2048 values per workgroup

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

// Exclusive scan of one 2048-value tile of in[gather[i]] (in[i] without gather).
// `block_sums` (if not null) receives the tile total; otherwise out[n] receives it.
__global__ __launch_bounds__(kScanThreads) void scan_tile_kernel(const uint32_t* __restrict__ in,
                                                                 const uint32_t* __restrict__ gather,
                                                                 uint32_t* __restrict__ out,
                                                                 int64_t n,
                                                                 uint32_t* __restrict__ block_sums) {
  __shared__ uint32_t s_v[kScanTile];
  __shared__ uint32_t s_wave[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int k = threadIdx.x; k < kScanTile; k += kScanThreads) {
    const int64_t idx = base + k;
    s_v[k] = idx < n ? in[gather ? gather[idx] : idx] : 0u;
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

// Sum of one 2048-value tile of in[gather[i]] (in[i] without gather) into block_sums[tile].
__global__ __launch_bounds__(kScanThreads) void scan_sum_kernel(const uint32_t* __restrict__ in,
                                                                const uint32_t* __restrict__ gather, int64_t n,
                                                                uint32_t* __restrict__ block_sums) {
  __shared__ uint32_t s_wave[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  uint32_t sum = 0;
#pragma unroll
  for (int e = 0; e < kScanItems; ++e) {
    const int64_t idx = base + e * kScanThreads + threadIdx.x;
    if (idx < n) sum += in[gather ? gather[idx] : idx];
  }
  uint32_t total;
  block_inclusive_scan(sum, s_wave, total);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// Exclusive scan of tile b of in[gather[i]], offset by the sum of the tiles before it (read
// from block_sums by the whole workgroup); the last tile also writes out[n].
__global__ __launch_bounds__(kScanThreads) void scan_tile_offset_kernel(const uint32_t* __restrict__ in,
                                                                        const uint32_t* __restrict__ gather,
                                                                        uint32_t* __restrict__ out, int64_t n,
                                                                        const uint32_t* __restrict__ block_sums) {
  __shared__ uint32_t s_v[kScanTile];
  __shared__ uint32_t s_wave[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int k = threadIdx.x; k < kScanTile; k += kScanThreads) {
    const int64_t idx = base + k;
    s_v[k] = idx < n ? in[gather ? gather[idx] : idx] : 0u;
  }
  uint32_t before = 0;
  for (int b = threadIdx.x; b < static_cast<int>(blockIdx.x); b += kScanThreads) before += block_sums[b];
  uint32_t prefix;
  block_inclusive_scan(before, s_wave, prefix);  // (the workgroup total of the partial sums)
  uint32_t local[kScanItems];
  uint32_t sum = 0;
#pragma unroll
  for (int e = 0; e < kScanItems; ++e) {
    local[e] = s_v[threadIdx.x * kScanItems + e];
    sum += local[e];
  }
  uint32_t total;
  const uint32_t incl = block_inclusive_scan(sum, s_wave, total);
  uint32_t run = prefix + incl - sum;
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
  if (threadIdx.x == 0 && blockIdx.x == gridDim.x - 1) out[n] = prefix + total;
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

// out[0] = sum of in[0..n) as a uint64: one workgroup of 1024 threads, 16-byte loads.
constexpr int kSumThreads = 1024;

__global__ __launch_bounds__(kSumThreads) void sum_u32_kernel(const uint32_t* __restrict__ in, int64_t n,
                                                              unsigned long long* __restrict__ out) {
  __shared__ unsigned long long s_w[kSumThreads / kWave];
  unsigned long long s = 0;
  const int64_t n4 = aligned16(in) ? n / 4 : 0;
  for (int64_t i = threadIdx.x; i < n4; i += kSumThreads) {
    const uint4 v = reinterpret_cast<const uint4*>(in)[i];
    s += static_cast<unsigned long long>(v.x) + v.y + v.z + v.w;
  }
  for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += kSumThreads) s += in[i];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long t = 0;
    for (int w = 0; w < kSumThreads / kWave; ++w) t += s_w[w];
    out[0] = t;
  }
}

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static size_t scan_ws(int64_t n) {
  if (n <= kScanTile) return 0;
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  return align_up(nb * 4) + align_up((nb + 1) * 4) + scan_ws(nb);
}

// Tiles up to which a scan is two launches (tile sums; each tile adds the sums before it to its
// own scan); beyond, the tile sums are scanned recursively (three launches per level).
constexpr int64_t kScanDirectTiles = 4096;

static void scan_rec(const uint32_t* in, uint32_t* out, int64_t n, char* ws, hipStream_t st,
                     const uint32_t* gather = nullptr) {
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  if (nb <= 1) {
    hipLaunchKernelGGL(scan_tile_kernel, dim3(1), dim3(kScanThreads), 0, st, in, gather, out, n, nullptr);
    return;
  }
  uint32_t* sums = reinterpret_cast<uint32_t*>(ws);
  if (nb <= kScanDirectTiles) {
    hipLaunchKernelGGL(scan_sum_kernel, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, st, in, gather, n,
                       sums);
    hipLaunchKernelGGL(scan_tile_offset_kernel, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, st, in,
                       gather, out, n, sums);
    return;
  }
  uint32_t* sums_scan = reinterpret_cast<uint32_t*>(ws + align_up(nb * 4));
  char* next = ws + align_up(nb * 4) + align_up((nb + 1) * 4);
  hipLaunchKernelGGL(scan_tile_kernel, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, st,
                     in, gather, out, n, sums);
  scan_rec(sums, sums_scan, nb, next, st);
  hipLaunchKernelGGL(scan_add_kernel, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, st,
                     out, n, sums_scan, nb);
}

// ---------------------------------------------------------------------------------------
// Small kernels
// ---------------------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void iota_u32_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = static_cast<uint32_t>(i);
}

__global__ void gather_u32_kernel(const uint32_t* __restrict__ src, const uint32_t* __restrict__ idx, int64_t n,
                                  uint32_t* __restrict__ out) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j < n) out[j] = src[idx[j]];
}

__global__ void fill_f32_kernel(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}



// ---------------------------------------------------------------------------------------
// Stable LSD radix sort of (uint32 key, uint32 value) pairs, BITS <= 8 bits per pass.
//
// Per pass three kernels, none of which waits on another workgroup:
//   upsweep  each 4096-key tile counts its digits (LDS atomics) -> tile_hist[digit][tile]
//   rowscan  one workgroup per digit: exclusive scan of its row over the tiles, and the
//            digit's total
//   scatter  each tile scans the digit totals (start of each digit), adds its row entries
//            -> global start of (digit, tile); ranks its keys stably (per-wavefront digit
//            counters in LDS; equal digits inside a 64-key round matched with BITS ballots),
//            stages the tile in LDS in digit order and writes it out as one contiguous run
//            per digit (coalesced)
// Wavefront w of a tile owns the contiguous keys [64 ROUNDS w, 64 ROUNDS (w + 1)), read in
// ROUNDS coalesced rounds, so (wavefront, round, lane) is input order: the sort is stable.
// ---------------------------------------------------------------------------------------
constexpr int kRsThreads = 256;
constexpr int kRsWaves = kRsThreads / kWave;      // 4
// A workgroup sorts a tile of 4 * 64 * ROUNDS keys; ROUNDS (4, 8 or 16) is chosen so that a
// sort has about 1000 tiles or more (enough workgroups to fill the chip).
constexpr int kRsMinTile = kRsWaves * kWave * 4;  // 1024 keys: smallest tile (sizes scratch)

template <int BITS>
__device__ __forceinline__ uint64_t match_bits(uint32_t d, bool valid) {
  uint64_t peers = __ballot(valid ? 1 : 0);
#pragma unroll
  for (int bit = 0; bit < BITS; ++bit) {
    const bool set = (d >> bit) & 1u;
    const uint64_t bm = __ballot(set ? 1 : 0);
    peers &= set ? bm : ~bm;
  }
  return valid ? peers : 0ull;
}


template <int BITS, int ROUNDS, typename K>
__global__ __launch_bounds__(kRsThreads) void rs_upsweep_kernel(const K* __restrict__ keys, int64_t m,
                                                                int shift, uint32_t* __restrict__ tile_hist,
                                                                int n_tiles) {
  constexpr int R = 1 << BITS;
  __shared__ uint32_t s_h[kRsWaves][R];  // per-wavefront counts (LDS atomics)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int k = threadIdx.x; k < kRsWaves * R; k += kRsThreads) (&s_h[0][0])[k] = 0;
  __syncthreads();
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t base = static_cast<int64_t>(tile) * (kRsWaves * kWave * ROUNDS) + wave * (kWave * ROUNDS);
  uint32_t key[ROUNDS];
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {  // all loads in flight before the first count
    const int64_t idx = base + r * kWave + lane;
    key[r] = idx < m ? keys[idx] : 0u;
  }
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    if (base + r * kWave + lane < m) atomicAdd(&s_h[wave][(key[r] >> shift) & (R - 1)], 1u);
  }
  __syncthreads();
  for (int k = threadIdx.x; k < R; k += kRsThreads) {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) c += s_h[w][k];
    tile_hist[static_cast<int64_t>(k) * n_tiles + tile] = c;
  }
}

// Workgroup `d`: entries [d][0 .. n_tiles) become the number of keys with digit d in earlier
// tiles; totals[d] receives the row total.
__global__ __launch_bounds__(kScanThreads) void rs_rowscan_kernel(uint32_t* __restrict__ tile_hist, int n_tiles,
                                                                  uint32_t* __restrict__ totals) {
  __shared__ uint32_t s_wave[4];
  const int d = blockIdx.x;
  uint32_t* row = tile_hist + static_cast<int64_t>(d) * n_tiles;
  uint32_t run = 0;
  for (int c0 = 0; c0 < n_tiles; c0 += kScanTile) {
    uint32_t loc[kScanItems];
    uint32_t sum = 0;
#pragma unroll
    for (int e = 0; e < kScanItems; ++e) {
      const int idx = c0 + static_cast<int>(threadIdx.x) * kScanItems + e;
      loc[e] = idx < n_tiles ? row[idx] : 0u;
      sum += loc[e];
    }
    uint32_t total;
    const uint32_t incl = block_inclusive_scan(sum, s_wave, total);
    uint32_t pos = run + incl - sum;
#pragma unroll
    for (int e = 0; e < kScanItems; ++e) {
      const int idx = c0 + static_cast<int>(threadIdx.x) * kScanItems + e;
      if (idx < n_tiles) row[idx] = pos;
      pos += loc[e];
    }
    run += total;
  }
  if (threadIdx.x == 0) totals[d] = run;
}

template <int BITS, int ROUNDS, typename K>
__global__ __launch_bounds__(kRsThreads) void rs_scatter_kernel(
    const K* __restrict__ kin, const uint32_t* __restrict__ vin, K* __restrict__ kout,
    uint32_t* __restrict__ vout, int64_t m, int shift, const uint32_t* __restrict__ tile_offs, int n_tiles,
    const uint32_t* __restrict__ totals, const uint32_t* __restrict__ aux_src, uint32_t* __restrict__ aux_out,
    uint32_t* __restrict__ ranges) {
  constexpr int R = 1 << BITS;
  __shared__ uint32_t s_cnt[kRsWaves][R];  // per-wavefront digit counts, then wavefront offsets
  __shared__ uint32_t s_excl[R];           // start of each digit inside the staged tile
  __shared__ uint32_t s_goff[R];           // global start of this tile's keys of each digit
  constexpr int kTileKeys = kRsWaves * kWave * ROUNDS;
  __shared__ uint32_t s_key[kTileKeys];
  __shared__ uint32_t s_val[kTileKeys];
  __shared__ uint32_t s_wave[4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  for (int k = threadIdx.x; k < kRsWaves * R; k += kRsThreads) (&s_cnt[0][0])[k] = 0;
  constexpr int DPT = (R + kRsThreads - 1) / kRsThreads;  // consecutive digits per thread (1 or 2)
  {
    // global start of (digit, tile): keys with a smaller digit + keys of the digit in earlier tiles
    uint32_t t[DPT], tsum = 0;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const int d = static_cast<int>(threadIdx.x) * DPT + e;
      t[e] = d < R ? totals[d] : 0u;
      tsum += t[e];
    }
    uint32_t all;
    uint32_t run = block_inclusive_scan(tsum, s_wave, all) - tsum;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const int d = static_cast<int>(threadIdx.x) * DPT + e;
      if (d < R) s_goff[d] = run + tile_offs[static_cast<int64_t>(d) * n_tiles + tile];
      run += t[e];
    }
  }
  __syncthreads();
  const int64_t tile_base = static_cast<int64_t>(tile) * kTileKeys;
  const int64_t base = tile_base + wave * (kWave * ROUNDS);
  const uint64_t lt = lanemask_lt(lane);
  uint32_t key[ROUNDS], val[ROUNDS], rank[ROUNDS];
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    const int64_t idx = base + r * kWave + lane;
    const bool valid = idx < m;
    key[r] = valid ? kin[idx] : 0u;
    val[r] = valid ? (vin ? vin[idx] : static_cast<uint32_t>(idx)) : 0u;
  }
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    const bool valid = base + r * kWave + lane < m;
    const uint32_t d = (key[r] >> shift) & (R - 1);
    const uint64_t peers = match_bits<BITS>(d, valid);
    rank[r] = valid ? s_cnt[wave][d] + static_cast<uint32_t>(__popcll(peers & lt)) : 0u;
    wave_sync();
    if (valid && (peers & lt) == 0ull) s_cnt[wave][d] += static_cast<uint32_t>(__popcll(peers));
    wave_sync();
  }
  __syncthreads();
  // digit totals of the tile -> wavefront offsets inside each digit, digit starts in the tile
  {
    uint32_t dt[DPT], tsum = 0;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const int d = static_cast<int>(threadIdx.x) * DPT + e;
      uint32_t acc = 0;
      if (d < R) {
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) {
          const uint32_t c = s_cnt[w][d];
          s_cnt[w][d] = acc;
          acc += c;
        }
      }
      dt[e] = acc;
      tsum += acc;
    }
    uint32_t all;
    uint32_t run = block_inclusive_scan(tsum, s_wave, all) - tsum;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const int d = static_cast<int>(threadIdx.x) * DPT + e;
      if (d < R) s_excl[d] = run;
      run += dt[e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    if (base + r * kWave + lane < m) {
      const uint32_t d = (key[r] >> shift) & (R - 1);
      const uint32_t pos = s_excl[d] + s_cnt[wave][d] + rank[r];
      s_key[pos] = key[r];
      s_val[pos] = val[r];
    }
  }
  __syncthreads();
  const int count = static_cast<int>(min<int64_t>(kTileKeys, m - tile_base));
  for (int p = threadIdx.x; p < count; p += kRsThreads) {
    const uint32_t k = s_key[p];
    const uint32_t d = (k >> shift) & (R - 1);
    const uint32_t g = s_goff[d] + (static_cast<uint32_t>(p) - s_excl[d]);
    if (kout) kout[g] = static_cast<K>(k);
    vout[g] = s_val[p];
    if (aux_out) aux_out[g] = aux_src[s_val[p]];  // a per-value array, gathered into sorted order
    if (ranges) {
      // last pass: the lower digits are sorted already, so a key's copies in this tile form one
      // run of consecutive output positions; the runs' ends give each key's [start, end) over
      // all tiles (ranges preset to [~0, 0])
      if (p == 0 || s_key[p - 1] != k) atomicMin(&ranges[2 * static_cast<int64_t>(k)], g);
      if (p == count - 1 || s_key[p + 1] != k) atomicMax(&ranges[2 * static_cast<int64_t>(k) + 1], g + 1u);
    }
  }
}

struct SortPlan {
  int passes, bits;
};

// Digits of at most kRsMaxBits bits (a 512-bin histogram per wavefront still fits LDS
// comfortably): 27-bit depth keys take 3 passes, 13-bit tile keys 2.
constexpr int kRsMaxBits = 9;
constexpr int kRsMaxPasses = 4;  // 32-bit keys

static SortPlan sort_plan(int bits) {
  SortPlan p;
  p.passes = bits <= 0 ? 0 : (bits + kRsMaxBits - 1) / kRsMaxBits;
  p.bits = p.passes ? (bits + p.passes - 1) / p.passes : 0;
  return p;
}

static size_t sort_ws(int64_t m) {
  const int64_t nt = (m + kRsMinTile - 1) / kRsMinTile;
  const int64_t hist = (int64_t(1) << kRsMaxBits) * (nt > 0 ? nt : 1);
  return align_up(m * 4) * 2 + align_up(hist * 4) + align_up(kRsMaxPasses * (1 << kRsMaxBits) * 4);
}

template <int BITS, int ROUNDS, typename K>
static void sort_pass_r(const K* sk, const uint32_t* sv, K* dk, uint32_t* dv, int64_t m, int shift,
                        uint32_t* tile_hist, int n_tiles, uint32_t* totals, hipStream_t st,
                        const uint32_t* aux_src, uint32_t* aux_out, uint32_t* ranges) {
  hipLaunchKernelGGL((rs_upsweep_kernel<BITS, ROUNDS, K>), dim3(n_tiles), dim3(kRsThreads), 0, st, sk, m, shift, tile_hist,
                     n_tiles);
  hipLaunchKernelGGL(rs_rowscan_kernel, dim3(1 << BITS), dim3(kScanThreads), 0, st, tile_hist, n_tiles, totals);
  hipLaunchKernelGGL((rs_scatter_kernel<BITS, ROUNDS, K>), dim3(n_tiles), dim3(kRsThreads), 0, st, sk, sv, dk, dv, m, shift,
                     tile_hist, n_tiles, totals, aux_src, aux_out, ranges);
}

static int sort_rounds(int64_t m) {
  if (m >= int64_t(1024) * 8192) return 16;
  if (m >= int64_t(1024) * 512) return 8;
  return 4;
}

template <int BITS, typename K>
static void sort_pass(const K* sk, const uint32_t* sv, K* dk, uint32_t* dv, int64_t m, int shift,
                      uint32_t* tile_hist, int rounds, uint32_t* totals, hipStream_t st, const uint32_t* aux_src,
                      uint32_t* aux_out, uint32_t* ranges) {
  const int n_tiles = static_cast<int>((m + kRsWaves * kWave * rounds - 1) / (kRsWaves * kWave * rounds));
  if (rounds == 16) sort_pass_r<BITS, 16>(sk, sv, dk, dv, m, shift, tile_hist, n_tiles, totals, st, aux_src, aux_out, ranges);
  else if (rounds == 8) sort_pass_r<BITS, 8>(sk, sv, dk, dv, m, shift, tile_hist, n_tiles, totals, st, aux_src, aux_out, ranges);
  else sort_pass_r<BITS, 4>(sk, sv, dk, dv, m, shift, tile_hist, n_tiles, totals, st, aux_src, aux_out, ranges);
}

// Sorts (k, v) by the low `bits` bits of k into (k_out, v_out), which must not alias (k, v).
// v = NULL stands for the values 0, 1, ..., m - 1.
// aux_src / aux_out (both or neither): the last pass also writes aux_out[j] = aux_src[v_out[j]].
// ranges (the sort has at least one pass): the last pass also takes every key value's [start,
// end) in the output by atomic min / max (ranges preset to [~0, 0]). drop_keys: the last pass
// writes only the values (k_out is still used by earlier passes). K: the key type (uint32_t, or
// uint16_t for keys below 2^16: a quarter fewer bytes per pass); the scratch is sized for 32-bit keys.
template <typename K>
static void radix_sort(const K* k, const uint32_t* v, K* k_out, uint32_t* v_out, int64_t m,
                       int bits, char* ws, hipStream_t st, const uint32_t* aux_src = nullptr,
                       uint32_t* aux_out = nullptr, uint32_t* ranges = nullptr, bool drop_keys = false) {
  if (m <= 0) return;
  const SortPlan plan = sort_plan(bits);
  if (plan.passes == 0) {
    (void)hipMemcpyAsync(k_out, k, m * sizeof(K), hipMemcpyDeviceToDevice, st);
    if (v) {
      (void)hipMemcpyAsync(v_out, v, m * 4, hipMemcpyDeviceToDevice, st);
    } else {
      hipLaunchKernelGGL(iota_u32_kernel, dim3(static_cast<unsigned>((m + 255) / 256)), dim3(256), 0, st, v_out, m);
    }
    if (aux_out)
      hipLaunchKernelGGL(gather_u32_kernel, dim3(static_cast<unsigned>((m + 255) / 256)), dim3(256), 0, st, aux_src,
                         v_out, m, aux_out);
    return;
  }
  const int rounds = sort_rounds(m);
  const int n_tiles = static_cast<int>((m + kRsMinTile - 1) / kRsMinTile);  // scratch sizing
  K* k_alt = reinterpret_cast<K*>(ws);
  ws += align_up(m * 4);
  uint32_t* v_alt = reinterpret_cast<uint32_t*>(ws);
  ws += align_up(m * 4);
  uint32_t* tile_hist = reinterpret_cast<uint32_t*>(ws);
  ws += align_up((static_cast<int64_t>(1) << kRsMaxBits) * n_tiles * 4);
  uint32_t* totals = reinterpret_cast<uint32_t*>(ws);
  // pass p writes the outputs when (passes - 1 - p) is even, the scratch pair otherwise, so
  // the last pass lands in (k_out, v_out) and no pass works in place
  const K* src_k = k;
  const uint32_t* src_v = v;
  for (int p = 0; p < plan.passes; ++p) {
    const bool to_out = ((plan.passes - 1 - p) % 2) == 0;
    K* dst_k = to_out ? k_out : k_alt;
    uint32_t* dst_v = to_out ? v_out : v_alt;
    uint32_t* tot = totals + (1 << kRsMaxBits) * p;
    const int shift = plan.bits * p;
    const bool last = p == plan.passes - 1;
    const uint32_t* as = last ? aux_src : nullptr;
    uint32_t* ao = last ? aux_out : nullptr;
    uint32_t* rg = last ? ranges : nullptr;
    K* dk = (last && drop_keys) ? nullptr : dst_k;
    switch (plan.bits) {
      case 1: sort_pass<1, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 2: sort_pass<2, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 3: sort_pass<3, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 4: sort_pass<4, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 5: sort_pass<5, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 6: sort_pass<6, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 7: sort_pass<7, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      case 8: sort_pass<8, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
      default: sort_pass<9, K>(src_k, src_v, dk, dst_v, m, shift, tile_hist, rounds, tot, st, as, ao, rg); break;
    }
    src_k = dst_k;
    src_v = dst_v;
  }
}

// ---------------------------------------------------------------------------------------
// Two-level binning: (1) stable sort of the Gaussians by depth key (culled ones last);
// (2) emission of (tile, Gaussian) instances in that order; (3) stable sort by tile.
// The result equals a stable sort of (tile << 32 | depth key) over instances emitted in
// Gaussian-index order.
// ---------------------------------------------------------------------------------------
// Depth sort keys. 3D: the view depth of the record, culled Gaussians last (the same keys
// gs_preprocess_fwd writes). 2D: the caller's depth (float32, or float64 split into a high
// and a low 32-bit key), every Gaussian kept, so the resulting order is the stable argsort of
// the depths.
__global__ void depth_keys_kernel(const SplatRec* __restrict__ rec, const float* __restrict__ depth,
                                  const double* __restrict__ depth64, const uint32_t* __restrict__ counts,
                                  int64_t n, uint32_t* __restrict__ keys, uint32_t* __restrict__ keys_hi) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t k = 0u;
  if (rec) {
    k = counts[i] != 0u ? float_order_key(rec[i].b.z) : 0xffffffffu;
  } else if (depth) {
    k = float_order_key(depth[i]);
  } else if (depth64) {
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(depth64[i] + 0.0));
    const uint64_t o = (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
    k = static_cast<uint32_t>(o);
    keys_hi[i] = static_cast<uint32_t>(o >> 32);
  }
  keys[i] = k;
}


// Tile rectangle (tx0, ty0, tx1, ty1), max exclusive, clipped to the tile grid.
__device__ __forceinline__ int4 clamp_rect(int4 r, int tiles_x, int tiles_y) {
  r.x = max(r.x, 0);
  r.y = max(r.y, 0);
  r.z = min(r.z, tiles_x);
  r.w = min(r.w, tiles_y);
  return r;
}

// 3D: tiles from the row-band rule; 2D: every tile of the rectangle [x0, x1) x [y0, y1).
// Emission is balanced by instances: wavefront w emits the Gaussians (in depth order) whose
// first instance lies in [kEmitSpan w, kEmitSpan (w + 1)), 64 at a time. The instances of 64
// consecutive Gaussians form one contiguous output range: the wavefront numbers their tile
// rows, computes the touched columns of up to kEmitChunk rows at a time (a lane per row), then
// writes rows of at least kEmitWide tiles one row at a time (a lane per tile) and the other
// rows' instances a lane per instance, so stores are coalesced.
constexpr uint32_t kEmitSpan = 256;
constexpr int kEmitChunk = 128;
constexpr int kEmitPer = kEmitChunk / kWave;  // rows per lane in the prefix step
constexpr uint32_t kEmitWide = 32;
constexpr int64_t kMaxTiles = int64_t(1) << 26;  // tile ids share a word with a 6-bit lane index

// First Gaussian of every emission window: Gaussian j starts the windows w with
// offs[j - 1] < kEmitSpan w <= offs[j]. wstart[n_windows] = the first Gaussian with
// offs[j] = m, which ends the last window (Gaussians after it have no instances).
__global__ void emit_windows_kernel(const uint32_t* __restrict__ offs, int64_t n, int64_t n_windows,
                                    uint32_t* __restrict__ wstart) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j > n) return;
  const int64_t cur = offs[j];
  const int64_t prev = j == 0 ? -1 : static_cast<int64_t>(offs[j - 1]);
  const int64_t w_lo = j == 0 ? 0 : prev / kEmitSpan + 1;
  const int64_t w_hi = min(cur / kEmitSpan, n_windows - 1);
  for (int64_t w = w_lo; w <= w_hi; ++w) wstart[w] = static_cast<uint32_t>(j);
  const int64_t m = offs[n];
  if (prev < m && cur >= m) wstart[n_windows] = static_cast<uint32_t>(j);
}

struct EmitSetup {
  float mx, my, invA, B, det, tA, vmax, vr;  // 3D band setup (what band_columns reads)
  int4 d;                                 // 3D: pixel bounds; rectangles: clamped tile rectangle
};

// Exclusive prefix sum over the wavefront; `total` receives the sum of all lanes.
__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v, int lane, uint32_t& total) {
  uint32_t incl = v;
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  total = __shfl(incl, kWave - 1, 64);
  return incl - v;
}

template <bool kRect, typename K>
__global__ __launch_bounds__(256) void emit_kernel(const SplatRec* __restrict__ rec,
                                                   const int4* __restrict__ rects,
                                                   const uint32_t* __restrict__ order,
                                                   const uint32_t* __restrict__ offs, int64_t n,
                                                   const uint32_t* __restrict__ wstart, int64_t n_windows,
                                                   int tiles_x, int tiles_y, K* __restrict__ tkeys,
                                                   uint32_t* __restrict__ vals, uint32_t* __restrict__ ranges_preset,
                                                   int n_tiles) {
  __shared__ EmitSetup s_set[4][kWave];
  __shared__ uint32_t s_rex[4][kWave];       // exclusive prefix of tile rows over the 64 Gaussians
  __shared__ uint32_t s_gid[4][kWave];
  __shared__ uint32_t s_iex[4][kEmitChunk];  // row instance counts, then their exclusive prefix
  __shared__ uint32_t s_nex[4][kEmitChunk];  // exclusive prefix over the narrow rows only
  __shared__ uint32_t s_row[4][kEmitChunk];  // (owner lane << 26) | first tile of the row
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (ranges_preset) {
    // [~0, 0] for every tile: the tile sort's last pass narrows them by atomic min / max
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < 2 * static_cast<int64_t>(n_tiles);
         q += stride)
      ranges_preset[q] = (q & 1) ? 0u : 0xffffffffu;
  }
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (w >= n_windows) return;  // whole wavefront
  const int64_t ja = wstart[w];
  const int64_t jb = wstart[w + 1];

  for (int64_t j0 = ja; j0 < jb; j0 += kWave) {
    const int64_t j = j0 + lane;
    uint32_t off = 0, cap = 0, rows = 0;
    if (j < jb) {
      off = offs[j];
      cap = offs[j + 1] - off;
    }
    EmitSetup es = {};
    uint32_t g = 0;
    if (cap) {
      g = order[j];
      if constexpr (kRect) {
        const int4 r = clamp_rect(rects[g], tiles_x, tiles_y);
        es.d = r;
        rows = (r.z > r.x && r.w > r.y) ? static_cast<uint32_t>(r.w - r.y) : 0u;
      } else {
        const float4 a = rec[g].a, b = rec[g].b;
        const int4 d = rec[g].d;
        const BandSetup bs = band_setup(a, b);
        es.mx = bs.mx; es.my = bs.my; es.invA = bs.invA; es.B = bs.B;
        es.det = bs.det; es.tA = bs.tA; es.vmax = bs.vmax; es.vr = bs.vr;
        es.d = d;
        rows = static_cast<uint32_t>(max(d.w / kTile - d.z / kTile + 1, 0));
      }
    }
    wave_sync();  // the previous group is done with the LDS
    s_set[wave][lane] = es;
    s_gid[wave][lane] = g;
    uint32_t total_rows;
    s_rex[wave][lane] = wave_excl_scan(rows, lane, total_rows);
    const uint32_t base = __shfl(off, 0, 64);
    const int last = static_cast<int>(min<int64_t>(kWave - 1, jb - 1 - j0));
    const uint32_t wave_cap = __shfl(off + cap, last, 64) - base;  // never write past the range
    wave_sync();

    uint32_t done = 0;
    for (uint32_t rc = 0; rc < total_rows; rc += kEmitChunk) {
      const int nr = static_cast<int>(min<uint32_t>(kEmitChunk, total_rows - rc));
      for (int q = lane; q < ((nr + kWave - 1) & ~(kWave - 1)); q += kWave) {
        uint32_t nt = 0, first = 0;
        if (q < nr) {
          const uint32_t item = rc + static_cast<uint32_t>(q);
          int own = 0;  // last Gaussian whose first row is <= item
#pragma unroll
          for (int step = 32; step > 0; step >>= 1)
            if (s_rex[wave][own + step] <= item) own += step;
          const EmitSetup& e = s_set[wave][own];
          const int r = static_cast<int>(item - s_rex[wave][own]);
          int ty, tx0;
          if constexpr (kRect) {
            ty = e.d.y + r;
            tx0 = e.d.x;
            nt = static_cast<uint32_t>(e.d.z - e.d.x);
          } else {
            BandSetup bs;
            bs.mx = e.mx; bs.my = e.my; bs.A = 0.0f; bs.invA = e.invA; bs.B = e.B;
            bs.det = e.det; bs.tA = e.tA; bs.vmax = e.vmax; bs.vr = e.vr;
            bs.ok = e.det > 0.0f;
            ty = e.d.z / kTile + r;
            nt = row_tiles(bs, e.d, ty, tx0);
          }
          first = (static_cast<uint32_t>(own) << 26) | static_cast<uint32_t>(ty * tiles_x + tx0);
        }
        s_iex[wave][q] = nt;
        s_row[wave][q] = first;
      }
      wave_sync();
      uint32_t c[kEmitPer], ex[kEmitPer], lsum = 0, nsum = 0;
#pragma unroll
      for (int e = 0; e < kEmitPer; ++e) {
        const int q = kEmitPer * lane + e;
        c[e] = q < nr ? s_iex[wave][q] : 0u;
        lsum += c[e];
        nsum += c[e] < kEmitWide ? c[e] : 0u;
      }
      uint32_t ctotal, ntotal;
      uint32_t run = wave_excl_scan(lsum, lane, ctotal);
      uint32_t nrun = wave_excl_scan(nsum, lane, ntotal);
      wave_sync();
#pragma unroll
      for (int e = 0; e < kEmitPer; ++e) {
        ex[e] = run;
        s_iex[wave][kEmitPer * lane + e] = run;
        s_nex[wave][kEmitPer * lane + e] = nrun;
        run += c[e];
        nrun += c[e] < kEmitWide ? c[e] : 0u;
      }
      wave_sync();
#pragma unroll
      for (int e = 0; e < kEmitPer; ++e) {
        for (uint64_t wm = __ballot(c[e] >= kEmitWide ? 1 : 0); wm != 0ull; wm &= wm - 1ull) {
          const int src = __ffsll(static_cast<unsigned long long>(wm)) - 1;
          const uint32_t nt = __shfl(c[e], src, 64), start = done + __shfl(ex[e], src, 64);
          const uint32_t rw = s_row[wave][kEmitPer * src + e];
          const uint32_t gw = s_gid[wave][rw >> 26];
          for (uint32_t t = lane; t < nt; t += kWave) {
            const uint32_t k = start + t;
            if (k < wave_cap) {
              tkeys[base + k] = static_cast<K>((rw & 0x3ffffffu) + t);
              vals[base + k] = gw;
            }
          }
        }
      }
      for (uint32_t p = lane; p < ntotal; p += kWave) {
        int q = 0;  // last row whose first narrow-row instance is <= p
#pragma unroll
        for (int step = kEmitChunk / 2; step > 0; step >>= 1)
          if (q + step < nr && s_nex[wave][q + step] <= p) q += step;
        const uint32_t rw = s_row[wave][q];
        const uint32_t t = p - s_nex[wave][q];
        const uint32_t k = done + s_iex[wave][q] + t;
        if (k < wave_cap) {
          tkeys[base + k] = static_cast<K>((rw & 0x3ffffffu) + t);
          vals[base + k] = s_gid[wave][rw >> 26];
        }
      }
      done += ctotal;
      wave_sync();
    }
  }
}

// Per-tile [start, end) of the sorted instances from the key changes: the instance that
// starts a tile writes its start (and gives the empty tiles before it the empty range at that
// position), the one that ends a tile writes its end (and closes the empty tiles after the
// last tile at m). Each thread takes kBoundsPer consecutive keys (16-byte loads). Used when
// the tile sort has no pass (a single tile); otherwise its last pass takes the ranges.
constexpr int kBoundsPer = 16;

__global__ __launch_bounds__(256) void tile_bounds_kernel(const uint32_t* __restrict__ tkeys, int64_t m,
                                                          int n_tiles, uint32_t* __restrict__ ranges) {
  const int64_t p0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * kBoundsPer;
  if (p0 >= m) return;
  uint32_t k[kBoundsPer + 2];  // k[0] = key p0 - 1, k[1 + e] = key p0 + e, k[kBoundsPer + 1] = key p0 + kBoundsPer
  const int cnt = static_cast<int>(min<int64_t>(kBoundsPer, m - p0));
  if (cnt == kBoundsPer) {
    const uint4* v = reinterpret_cast<const uint4*>(tkeys + p0);
#pragma unroll
    for (int q = 0; q < kBoundsPer / 4; ++q) {
      const uint4 x = v[q];
      k[1 + 4 * q] = x.x;
      k[2 + 4 * q] = x.y;
      k[3 + 4 * q] = x.z;
      k[4 + 4 * q] = x.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < kBoundsPer; ++e) k[1 + e] = e < cnt ? tkeys[p0 + e] : 0u;
  }
  k[0] = p0 > 0 ? tkeys[p0 - 1] : 0u;
  k[kBoundsPer + 1] = p0 + kBoundsPer < m ? tkeys[p0 + kBoundsPer] : 0u;
  for (int e = 0; e < kBoundsPer; ++e) {
    if (e >= cnt) break;
    const int64_t p = p0 + e;
    const uint32_t t = k[1 + e];
    if (t >= static_cast<uint32_t>(n_tiles)) continue;  // not a tile id
    const uint32_t pos = static_cast<uint32_t>(p);
    const uint32_t prev = k[e];
    if (p == 0 || prev != t) {
      const uint32_t lo = p == 0 ? 0u : (prev < t ? prev + 1u : t);
      for (uint32_t u = lo; u < t; ++u) {
        ranges[2 * u] = pos;
        ranges[2 * u + 1] = pos;
      }
      ranges[2 * t] = pos;
    }
    const bool last = p == m - 1;
    if (last || k[2 + e] != t) {
      ranges[2 * t + 1] = pos + 1u;
      if (last) {
        for (uint32_t u = t + 1u; u < static_cast<uint32_t>(n_tiles); ++u) {
          ranges[2 * u] = pos + 1u;
          ranges[2 * u + 1] = pos + 1u;
        }
      }
    }
  }
}

// One workgroup: bucket counts ceil(len / 32) per tile, their exclusive scan into
// bucket_offsets [T + 1], and optionally the CSR tile offsets [T + 1]. With m == 0 it also
// writes the (empty) ranges.
constexpr int kBoThreads = 1024;
constexpr int kBoItems = 8;

__global__ __launch_bounds__(kBoThreads) void bucket_offsets_kernel(uint32_t* __restrict__ ranges, int n_tiles,
                                                                    int64_t m, uint32_t* __restrict__ boff,
                                                                    uint32_t* __restrict__ tile_offsets,
                                                                    uint32_t* __restrict__ list_header,
                                                                    bool fix_empty) {
  __shared__ uint32_t s_wave[kBoThreads / kWave];
  __shared__ uint32_t s_wave_inst[kBoThreads / kWave];
  if (list_header && threadIdx.x < kListHeader) list_header[threadIdx.x] = 0u;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // fix_empty: ranges come from the sort's atomic min / max, so a tile without instances still
  // holds [~0, 0]; the instance counts are scanned beside the bucket counts and such a tile gets
  // the empty range at its CSR position
  uint32_t run = 0, run_inst = 0;
  for (int c0 = 0; c0 < n_tiles; c0 += kBoThreads * kBoItems) {
    uint32_t cnt[kBoItems], start[kBoItems], len[kBoItems], sum = 0, sum_inst = 0;
#pragma unroll
    for (int e = 0; e < kBoItems; ++e) {
      const int t = c0 + static_cast<int>(threadIdx.x) * kBoItems + e;
      cnt[e] = 0;
      start[e] = 0;
      len[e] = 0;
      if (t < n_tiles) {
        if (m > 0) {
          start[e] = ranges[2 * t];
          const uint32_t end = ranges[2 * t + 1];
          len[e] = (fix_empty && start[e] == 0xffffffffu) ? 0u : end - start[e];
          cnt[e] = (len[e] + kBucket - 1) / kBucket;
        } else {
          ranges[2 * t] = 0;
          ranges[2 * t + 1] = 0;
        }
      }
      sum += cnt[e];
      sum_inst += len[e];
    }
    uint32_t incl = sum, incl_inst = sum_inst;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const uint32_t u = __shfl_up(incl, o, 64);
      const uint32_t ui = __shfl_up(incl_inst, o, 64);
      if (lane >= o) {
        incl += u;
        incl_inst += ui;
      }
    }
    if (lane == kWave - 1) {
      s_wave[wave] = incl;
      s_wave_inst[wave] = incl_inst;
    }
    __syncthreads();
    uint32_t before = 0, total = 0, before_inst = 0, total_inst = 0;
    for (int w = 0; w < kBoThreads / kWave; ++w) {
      const uint32_t v = s_wave[w];
      const uint32_t vi = s_wave_inst[w];
      before += w < wave ? v : 0u;
      before_inst += w < wave ? vi : 0u;
      total += v;
      total_inst += vi;
    }
    __syncthreads();
    uint32_t pos = run + before + incl - sum;
    uint32_t pos_inst = run_inst + before_inst + incl_inst - sum_inst;
#pragma unroll
    for (int e = 0; e < kBoItems; ++e) {
      const int t = c0 + static_cast<int>(threadIdx.x) * kBoItems + e;
      if (t < n_tiles) {
        boff[t] = pos;
        if (fix_empty && m > 0 && len[e] == 0) {
          start[e] = pos_inst;
          ranges[2 * t] = pos_inst;
          ranges[2 * t + 1] = pos_inst;
        }
        if (tile_offsets) tile_offsets[t] = start[e];
      }
      pos += cnt[e];
      pos_inst += len[e];
    }
    run += total;
    run_inst += total_inst;
  }
  if (threadIdx.x == 0) {
    boff[n_tiles] = run;
    if (tile_offsets) tile_offsets[n_tiles] = static_cast<uint32_t>(m);
  }
}

// Full 64-bit keys of the sorted instances (tile << 32 | depth key), for callers that want them.
// (tile << 32 | depth order key); dkey0 is added back to keys stored relative to it.
template <typename K>
__global__ void full_keys_kernel(const K* __restrict__ tkeys, const uint32_t* __restrict__ vals,
                                 const uint32_t* __restrict__ dkey_of, uint32_t dkey0, int64_t m,
                                 uint64_t* __restrict__ out) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p < m) out[p] = (static_cast<uint64_t>(tkeys[p]) << 32) | (dkey_of[vals[p]] + dkey0);
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

__global__ void rect_counts_kernel(const int4* __restrict__ rects, int64_t n, int tiles_x, int tiles_y,
                                   uint32_t* __restrict__ counts) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int4 r = clamp_rect(rects[i], tiles_x, tiles_y);
  const int w = r.z - r.x, h = r.w - r.y;
  counts[i] = (w > 0 && h > 0) ? static_cast<uint32_t>(w * h) : 0u;
}

static inline unsigned grid_for(int64_t n, int threads) {
  return static_cast<unsigned>((n + threads - 1) / threads);
}

static int bits_for(int64_t n_values) {
  int b = 0;
  while ((int64_t(1) << b) < n_values) ++b;
  return b;
}

// Workspace layouts, as byte offsets from the start of the workspace. The size functions
// below return a layout's `end`, and the code that carves a workspace takes its regions from
// the same layout, so the two cannot disagree.
//
// Depth ordering: keys, sorted keys, float64 high keys (then the counts in depth order),
// temporary values, sort scratch, scan scratch.
struct PrepLayout {
  size_t dkeys, dsorted, khi, tmpv, sort, scan, end;
};

static PrepLayout prep_layout(int64_t n) {
  PrepLayout L;
  size_t o = 0;
  L.dkeys = o; o += align_up(n * 4);
  L.dsorted = o; o += align_up(n * 4);
  L.khi = o; o += align_up(n * 4);
  L.tmpv = o; o += align_up(n * 4);
  L.sort = o; o += sort_ws(n);
  L.scan = o; o += scan_ws(n);
  L.end = o;
  return L;
}

// Emission and tile sort: tile keys and values, sorted tile keys, sort scratch, window starts.
struct EmitLayout {
  size_t tkeys, tvals, tsorted, sort, wstart, end;
  int tile_bits;
};

static EmitLayout emit_layout(int64_t m, int n_tiles) {
  EmitLayout L;
  L.tile_bits = bits_for(n_tiles);
  size_t o = 0;
  L.tkeys = o; o += align_up(m * 4);
  L.tvals = o; o += align_up(m * 4);
  L.tsorted = o; o += align_up(m * 4);
  L.sort = o; o += sort_ws(m);
  L.wstart = o; o += align_up(static_cast<size_t>((m + kEmitSpan - 1) / kEmitSpan + 1) * 4);
  L.end = o;
  return L;
}

// Rectangle binning: the depth ordering, the order and offsets, then the emission.
struct RectLayout {
  size_t prep, order, offs, emit, end;
};

static RectLayout rect_layout(int64_t n, int64_t m, int n_tiles) {
  RectLayout L;
  size_t o = 0;
  L.prep = o; o += prep_layout(n).end;
  L.order = o; o += align_up(n * 4);
  L.offs = o; o += align_up((n + 1) * 4);
  L.emit = o; o += emit_layout(m, n_tiles).end;
  L.end = o;
  return L;
}

static size_t prep_ws(int64_t n) { return prep_layout(n).end; }
static size_t emit_ws(int64_t m, int n_tiles) { return emit_layout(m, n_tiles).end; }

// Stable order of the Gaussians by depth key (keys_in: precomputed 32-bit keys, else computed
// from rec / depth / depth64; none of them: index order) and, if offsets is not NULL, the
// exclusive scan of their instance counts in that order (offsets[n] = m).
static void bin_prepare(const SplatRec* rec, const float* depth, const double* depth64, const uint32_t* keys_in,
                        int key_bits, const uint32_t* counts, int64_t n, uint32_t* order, uint32_t* offsets,
                        char* ws, hipStream_t st) {
  const PrepLayout L = prep_layout(n);
  uint32_t* dkeys = reinterpret_cast<uint32_t*>(ws + L.dkeys);
  uint32_t* dsorted = reinterpret_cast<uint32_t*>(ws + L.dsorted);
  uint32_t* khi = reinterpret_cast<uint32_t*>(ws + L.khi);
  uint32_t* tmpv = reinterpret_cast<uint32_t*>(ws + L.tmpv);
  char* sort_scratch = ws + L.sort;
  char* scan_scratch = ws + L.scan;
  if (n <= 0) {
    if (offsets) hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, st, offsets, int64_t(1), 0u);
    return;
  }
  if (keys_in || rec || depth || depth64) {
    const uint32_t* keys = keys_in;
    int bits = keys_in ? key_bits : 32;
    if (!keys) {
      hipLaunchKernelGGL(depth_keys_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, rec, depth, depth64,
                         counts, n, dkeys, depth64 ? khi : nullptr);
      keys = dkeys;
    }
    // the final pass also writes the counts in depth order (into khi, free by then), so the scan
    // reads them contiguously instead of through the order; the sorted keys themselves are not
    // needed, so it writes none
    uint32_t* sorted_counts = offsets ? khi : nullptr;
    if (depth64) {
      // low key halves first, then stably by the high halves gathered into that order
      radix_sort(keys, nullptr, dsorted, tmpv, n, 32, sort_scratch, st);
      hipLaunchKernelGGL(gather_u32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, khi, tmpv, n, dkeys);
      radix_sort(dkeys, tmpv, dsorted, order, n, 32, sort_scratch, st, sorted_counts ? counts : nullptr,
                 sorted_counts, nullptr, true);
    } else {
      radix_sort(keys, nullptr, dsorted, order, n, bits, sort_scratch, st, sorted_counts ? counts : nullptr,
                 sorted_counts, nullptr, true);
    }
    if (offsets) scan_rec(sorted_counts, offsets, n, scan_scratch, st);
  } else {
    hipLaunchKernelGGL(iota_u32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, order, n);
    if (offsets) scan_rec(counts, offsets, n, scan_scratch, st);  // index order
  }
}

// Emission of the instances in depth order, stable sort by tile, tile ranges and bucket
// offsets. dkey_of [n]: the depth key of every Gaussian (only read for sorted_keys).
// Emission and the stable tile sort with keys of type K (the ranges preset by the emission
// and taken by the last pass when there is one), and the full 64-bit keys if asked for.
template <typename K>
static void emit_and_sort(const SplatRec* rec, const int4* rects, const uint32_t* dkey_of, uint32_t dkey0,
                          const uint32_t* order, const uint32_t* offsets, int64_t n, int tiles_x, int n_tiles,
                          int64_t m, int tile_bits, uint64_t* sorted_keys, uint32_t* point_list, uint32_t* preset,
                          const EmitLayout& L, char* ws, hipStream_t st) {
  K* tkeys = reinterpret_cast<K*>(ws + L.tkeys);
  uint32_t* tvals = reinterpret_cast<uint32_t*>(ws + L.tvals);
  K* tsorted = reinterpret_cast<K*>(ws + L.tsorted);
  const uint32_t* wstart = reinterpret_cast<const uint32_t*>(ws + L.wstart);
  const int64_t n_windows = (m + kEmitSpan - 1) / kEmitSpan;
  if (rects) {
    hipLaunchKernelGGL((emit_kernel<true, K>), dim3(grid_for(n_windows, 4)), dim3(256), 0, st, rec, rects, order,
                       offsets, n, wstart, n_windows, tiles_x, n_tiles / tiles_x, tkeys, tvals, preset, n_tiles);
  } else {
    hipLaunchKernelGGL((emit_kernel<false, K>), dim3(grid_for(n_windows, 4)), dim3(256), 0, st, rec, rects, order,
                       offsets, n, wstart, n_windows, tiles_x, n_tiles / tiles_x, tkeys, tvals, preset, n_tiles);
  }
  radix_sort(tkeys, tvals, tsorted, point_list, m, tile_bits, ws + L.sort, st, nullptr, nullptr, preset,
             preset != nullptr && !sorted_keys);
  if (sorted_keys)
    hipLaunchKernelGGL((full_keys_kernel<K>), dim3(grid_for(m, 256)), dim3(256), 0, st, tsorted, point_list, dkey_of,
                       dkey0, m, sorted_keys);
}

static void bin_emit(const SplatRec* rec, const int4* rects, const uint32_t* dkey_of, uint32_t dkey0,
                     const uint32_t* order,
                     const uint32_t* offsets, int64_t n, int tiles_x, int n_tiles, int64_t m,
                     uint64_t* sorted_keys, uint32_t* point_list, uint32_t* ranges, uint32_t* tile_offsets,
                     uint32_t* bucket_offsets, uint32_t* list_header, char* ws, hipStream_t st) {
  const EmitLayout L = emit_layout(m, n_tiles);
  const int tile_bits = L.tile_bits;
  if (m > 0) {
    const int64_t n_windows = (m + kEmitSpan - 1) / kEmitSpan;
    hipLaunchKernelGGL(emit_windows_kernel, dim3(grid_for(n + 1, 256)), dim3(256), 0, st, offsets, n, n_windows,
                       reinterpret_cast<uint32_t*>(ws + L.wstart));
    // with at least one sort pass, the last pass takes the tile ranges (preset by the emission)
    // and the sorted keys are written only if the caller wants them; tile ids below 2^16 are
    // emitted and sorted as 16-bit keys
    const bool sort_ranges = tile_bits > 0;
    uint32_t* preset = sort_ranges ? ranges : nullptr;
    if (sort_ranges && n_tiles <= 65536)
      emit_and_sort<uint16_t>(rec, rects, dkey_of, dkey0, order, offsets, n, tiles_x, n_tiles, m, tile_bits,
                              sorted_keys, point_list, preset, L, ws, st);
    else
      emit_and_sort<uint32_t>(rec, rects, dkey_of, dkey0, order, offsets, n, tiles_x, n_tiles, m, tile_bits,
                              sorted_keys, point_list, preset, L, ws, st);
    if (!sort_ranges)
      hipLaunchKernelGGL(tile_bounds_kernel, dim3(grid_for((m + kBoundsPer - 1) / kBoundsPer, 256)), dim3(256), 0,
                         st, reinterpret_cast<const uint32_t*>(ws + L.tsorted), m, n_tiles, ranges);
    hipLaunchKernelGGL(bucket_offsets_kernel, dim3(1), dim3(kBoThreads), 0, st, ranges, n_tiles, m, bucket_offsets,
                       tile_offsets, list_header, sort_ranges);
    return;
  }
  hipLaunchKernelGGL(bucket_offsets_kernel, dim3(1), dim3(kBoThreads), 0, st, ranges, n_tiles, m, bucket_offsets,
                     tile_offsets, list_header, false);
}

}  // namespace gs

using namespace gs;

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

extern "C" int gs_sum_u32(const uint32_t* in, int64_t n, uint64_t* out, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && out && (n == 0 || in), GS_ERR_ARG, "invalid sum arguments");
  GS_REQUIRE(aligned(in, 4) && aligned(out, 8), GS_ERR_ALIGN, "sum: 4-byte aligned input, 8-byte aligned output");
  hipLaunchKernelGGL(sum_u32_kernel, dim3(1), dim3(kSumThreads), 0, as_stream(stream), in, n,
                     reinterpret_cast<unsigned long long*>(out));
  return check_launch("sum_u32");
}

extern "C" size_t gs_bin_prepare_workspace_size(int64_t n) { return prep_ws(n < 0 ? 0 : n); }

extern "C" int gs_bin_prepare_3d(const float* splat_rec, const uint32_t* tiles_touched,
                                 const uint32_t* depth_keys, int64_t n, const gs_camera* cam, uint32_t* order,
                                 uint32_t* offsets, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (int e = check_cam(cam)) return e;
  GS_REQUIRE(n >= 0 && n < (int64_t(1) << 32) && offsets, GS_ERR_ARG, "invalid bin_prepare arguments");
  GS_REQUIRE(n == 0 || (tiles_touched && order && (depth_keys || splat_rec)), GS_ERR_ARG,
             "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16), GS_ERR_ALIGN, "splat_rec must be 16-byte aligned");
  const size_t need = prep_ws(n);
  GS_REQUIRE(workspace_bytes >= need && workspace, GS_ERR_WORKSPACE,
             "bin_prepare workspace too small: need %zu bytes", need);
  bin_prepare(depth_keys ? nullptr : reinterpret_cast<const SplatRec*>(splat_rec), nullptr, nullptr, depth_keys,
              depth_key_bits(make_cam(*cam)), tiles_touched, n, order, offsets, static_cast<char*>(workspace),
              as_stream(stream));
  return check_launch("bin_prepare_3d");
}

extern "C" size_t gs_bin_workspace_size(int64_t n, int64_t m, int n_tiles) {
  n = n < 0 ? 0 : n;
  n_tiles = n_tiles < 1 ? 1 : n_tiles;
  m = m < 0 ? 0 : m;
  // the rectangle binning runs the depth ordering itself: its scratch, order and offsets too
  return rect_layout(n, m, n_tiles).end;
}

extern "C" int gs_bin_fill_3d(const float* splat_rec, const uint32_t* depth_keys, const uint32_t* order,
                              const uint32_t* offsets, int64_t n, const gs_camera* cam, int64_t m,
                              uint64_t* sorted_keys, uint32_t* point_list, uint32_t* ranges,
                              uint32_t* bucket_offsets, uint32_t* bucket_list, void* workspace,
                              size_t workspace_bytes, void* stream) {
  clear_error();
  if (int e = check_cam(cam)) return e;
  GS_REQUIRE(n >= 0 && m >= 0 && m < (int64_t(1) << 32), GS_ERR_ARG, "invalid sizes n=%lld m=%lld",
             static_cast<long long>(n), static_cast<long long>(m));
  GS_REQUIRE(ranges && bucket_offsets, GS_ERR_ARG, "null output");
  const CamK k = make_cam(*cam);
  GS_REQUIRE(static_cast<int64_t>(k.tiles_x) * k.tiles_y < kMaxTiles, GS_ERR_ARG, "too many tiles");
  const int n_tiles = k.tiles_x * k.tiles_y;
  const size_t need = emit_ws(m, n_tiles);
  GS_REQUIRE(workspace_bytes >= need && workspace, GS_ERR_WORKSPACE,
             "binning workspace too small: need %zu bytes", need);
  GS_REQUIRE(m == 0 || (splat_rec && order && offsets && point_list), GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(!(sorted_keys && m > 0 && !depth_keys), GS_ERR_ARG, "sorted_keys need depth_keys");
  GS_REQUIRE(aligned(splat_rec, 16), GS_ERR_ALIGN, "splat_rec must be 16-byte aligned");
  bin_emit(reinterpret_cast<const SplatRec*>(splat_rec), nullptr, depth_keys, k.dkey0, order, offsets, n, k.tiles_x,
           n_tiles,
           m, sorted_keys, point_list, ranges, nullptr, bucket_offsets, bucket_list, static_cast<char*>(workspace),
           as_stream(stream));
  return check_launch("bin_fill_3d");
}

extern "C" int gs_rect_counts(const int32_t* rects, int64_t n, int tiles_x, int tiles_y, uint32_t* counts,
                              void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && (n == 0 || (rects && counts)) && tiles_x > 0 && tiles_y > 0, GS_ERR_ARG,
             "invalid rect_counts arguments");
  GS_REQUIRE(aligned(rects, 16), GS_ERR_ALIGN, "rects must be 16-byte aligned");
  if (n == 0) return GS_OK;
  hipLaunchKernelGGL(rect_counts_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const int4*>(rects), n, tiles_x, tiles_y, counts);
  return check_launch("rect_counts");
}

extern "C" int gs_bin_fill_rect(const int32_t* rects, const void* depth, int depth_dtype,
                                const uint32_t* counts, int64_t n, int tiles_x, int tiles_y, int64_t m,
                                uint64_t* sorted_keys, uint32_t* point_list, uint32_t* ranges,
                                uint32_t* tile_offsets, uint32_t* bucket_offsets, uint32_t* order,
                                void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && m >= 0 && m < (int64_t(1) << 32) && tiles_x > 0 && tiles_y > 0, GS_ERR_ARG,
             "invalid sizes");
  GS_REQUIRE(static_cast<int64_t>(tiles_x) * tiles_y < kMaxTiles, GS_ERR_ARG, "too many tiles");
  GS_REQUIRE(depth_dtype == GS_FLOAT32 || depth_dtype == GS_FLOAT64, GS_ERR_ARG, "invalid depth dtype");
  GS_REQUIRE(ranges && bucket_offsets, GS_ERR_ARG, "null output");
  const int n_tiles = tiles_x * tiles_y;
  const size_t need = gs_bin_workspace_size(n, m, n_tiles);
  GS_REQUIRE(workspace_bytes >= need && workspace, GS_ERR_WORKSPACE,
             "binning workspace too small: need %zu bytes", need);
  GS_REQUIRE(m == 0 || (rects && counts && point_list), GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(!(depth && depth_dtype == GS_FLOAT64 && sorted_keys), GS_ERR_ARG,
             "sorted_keys are 32-bit depth keys: not available with a float64 depth");
  GS_REQUIRE(aligned(rects, 16), GS_ERR_ALIGN, "rects must be 16-byte aligned");
  const float* d32 = depth_dtype == GS_FLOAT32 ? static_cast<const float*>(depth) : nullptr;
  const double* d64 = depth_dtype == GS_FLOAT64 ? static_cast<const double*>(depth) : nullptr;
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  const RectLayout L = rect_layout(n, m, n_tiles);
  char* prep = ws + L.prep;
  uint32_t* dkeys = reinterpret_cast<uint32_t*>(prep + prep_layout(n).dkeys);
  uint32_t* ord = order ? order : reinterpret_cast<uint32_t*>(ws + L.order);
  uint32_t* offs = reinterpret_cast<uint32_t*>(ws + L.offs);
  if (n > 0 && (m > 0 || order)) {
    bin_prepare(nullptr, d32, d64, nullptr, 32, counts, n, ord, m > 0 ? offs : nullptr, prep, st);
    if (sorted_keys && m > 0 && !d32)  // index order: the depth part of the keys is 0
      hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, dkeys, n, 0u);
  }
  bin_emit(nullptr, reinterpret_cast<const int4*>(rects), dkeys, 0u, ord, offs, n, tiles_x, n_tiles, m, sorted_keys,
           point_list, ranges, tile_offsets, bucket_offsets, nullptr, ws + L.emit, st);
  return check_launch("bin_fill_rect");
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
