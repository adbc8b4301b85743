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
  // depth keys (more than 16 bits) from 2M keys on take 4096-key tiles: 3M SH3 depth order 140 ->
  // 131 us (at 1M the 2048-key tiles are faster, 74 against 80 us; the 16-bit tile keys keep
  // sort_rounds' tiles, measured best for them up to 8M)
  const int rounds = (bits > 16 && m >= int64_t(1024) * 2048) ? 16 : sort_rounds(m);
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

// Wavefronts per workgroup of emit_kernel: one. Each takes its own window and shares nothing with
// the others (1M SH3 key duplication 41.4 -> 40.5 us against four per workgroup).
constexpr int kEmitWaves = 1;
template <bool kRect, typename K>
__global__ __launch_bounds__(kEmitWaves * 64) void emit_kernel(const SplatRec* __restrict__ rec,
                                                   const int4* __restrict__ rects,
                                                   const uint32_t* __restrict__ order,
                                                   const uint32_t* __restrict__ offs, int64_t n,
                                                   const uint32_t* __restrict__ wstart, int64_t n_windows,
                                                   int tiles_x, int tiles_y, K* __restrict__ tkeys,
                                                   uint32_t* __restrict__ vals, uint32_t* __restrict__ ranges_preset,
                                                   int n_tiles) {
  __shared__ EmitSetup s_set[kEmitWaves][kWave];
  __shared__ uint32_t s_rex[kEmitWaves][kWave];       // exclusive prefix of tile rows over the 64 Gaussians
  __shared__ uint32_t s_gid[kEmitWaves][kWave];
  __shared__ uint32_t s_iex[kEmitWaves][kEmitChunk];  // row instance counts, then their exclusive prefix
  __shared__ uint32_t s_nex[kEmitWaves][kEmitChunk];  // exclusive prefix over the narrow rows only
  __shared__ uint32_t s_row[kEmitWaves][kEmitChunk];  // (owner lane << 26) | first tile of the row
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (ranges_preset) {
    // [~0, 0] for every tile: the tile sort's last pass narrows them by atomic min / max
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < 2 * static_cast<int64_t>(n_tiles);
         q += stride)
      ranges_preset[q] = (q & 1) ? 0u : 0xffffffffu;
  }
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kEmitWaves + wave;
  if (w >= n_windows) return;  // whole wavefront
  const int64_t ja = wstart[w];
  const int64_t jb = wstart[w + 1];

  for (int64_t j0 = ja; j0 < jb; j0 += kWave) {
    const int64_t j = j0 + lane;
    uint32_t off = 0, cap = 0, rows = 0, gj = 0;
    if (j < jb) {
      // (the Gaussian's id is loaded beside its offsets, not after them)
      gj = order ? order[j] : static_cast<uint32_t>(j);
      off = offs[j];
      cap = offs[j + 1] - off;
    }
    EmitSetup es = {};
    uint32_t g = 0;
    if (cap) {
      g = gj;
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

// ---------------------------------------------------------------------------------------
// Span binning (canvases of at most kSpanMaxDim tiles per side).
//
// The tile lists in (tile, depth) order without sorting the M instances. A Gaussian's tiles
// in one tile row form a run of columns, its row span (tx0, nt); two counting passes over the
// spans place every instance once:
//   rows     the Gaussians in depth order, kRowChunk per wavefront: each chunk counts its
//            non-empty (Gaussian, tile row) items per row (span_rows_kernel<count>), a scan of
//            each row over the chunks gives every chunk its offsets (rs_rowscan_kernel), and
//            each chunk writes its spans there (span_rows_kernel<write>): the spans of one row
//            are contiguous and in depth order. Each row's spans start at a multiple of
//            kSpanChunk.
//   columns  kSpanChunk spans per wavefront, all of one row: each chunk counts its instances
//            per column with a difference array over the columns (span_col_count_kernel); a
//            scan of every (row, column) over the row's chunks gives every chunk its offsets
//            and the tile counts, and the last workgroup to finish scans the tile counts into
//            ranges and bucket offsets (span_col_scan_kernel); each chunk expands its spans into
//            instances and writes the Gaussian of each at its tile's start + the chunk's offset
//            + its rank among the chunk's instances in that column (span_col_write_kernel).
// Ranks inside a wavefront come from ballots over the row or column bits in item order, and
// chunks keep their order through the scans, so both passes are stable and a tile's list
// holds its Gaussians in depth order: the order of a stable sort by tile of the instances
// emitted in depth order. No kernel waits on another workgroup.
// ---------------------------------------------------------------------------------------
constexpr int kSpanMaxDim = 512;   // tiles per side (the LDS of the placement kernels)
constexpr int kRowChunk = 256;     // depth positions per wavefront in the row pass
constexpr int kSpanChunk = 1024;   // spans per workgroup in the column pass
constexpr int kSpanWaves = 4;      // wavefronts per workgroup (256 threads)
constexpr int kColScanThreads = kBoThreads;  // the last workgroup runs tile_scan_block

__device__ __forceinline__ int align4i(int v) { return (v + 3) & ~3; }

__device__ __forceinline__ uint32_t span_pad(uint32_t v) {
  return (v + kSpanChunk - 1) & ~static_cast<uint32_t>(kSpanChunk - 1);
}

// s_rbase[r], r = 0 .. tiles_y: the start of row r's spans, every row's span count rounded up
// to a multiple of kSpanChunk (s_rbase[tiles_y] = all of them). Called by every thread of the
// workgroup; ends with a barrier. s_wsum: one word per wavefront.
template <int kThreads>
__device__ void span_row_bases(const uint32_t* __restrict__ rowtot, int tiles_y, uint32_t* s_rbase,
                               uint32_t* s_wsum) {
  constexpr int kPer = (kSpanMaxDim + 1 + kThreads - 1) / kThreads;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t v[kPer], sum = 0;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int r = static_cast<int>(threadIdx.x) * kPer + e;
    v[e] = r < tiles_y ? span_pad(rowtot[r]) : 0u;
    sum += v[e];
  }
  uint32_t incl = sum;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == kWave - 1) s_wsum[wave] = incl;
  __syncthreads();
  uint32_t run = incl - sum;
  for (int w = 0; w < wave; ++w) run += s_wsum[w];
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int r = static_cast<int>(threadIdx.x) * kPer + e;
    if (r <= tiles_y) s_rbase[r] = run;
    run += v[e];
  }
  __syncthreads();
}

// The row whose spans hold position p: the largest r < tiles_y with s_rbase[r] <= p.
__device__ __forceinline__ int span_row_of(const uint32_t* s_rbase, int tiles_y, uint32_t p) {
  int lo = 0, hi = tiles_y - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_rbase[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// The span of item `item` of a wavefront's 64 Gaussians (their band setups or rectangles in
// s_set, the exclusive prefix of their row counts in s_rex): the owning Gaussian (lane index),
// the tile row and first column; returns the number of tiles (0: the row is missed).
template <bool kRect>
__device__ __forceinline__ uint32_t row_item(const float4* s_set, const uint32_t* s_rex, uint32_t item, int& own,
                                             int& row, uint32_t& tx0) {
  own = 0;  // last Gaussian whose first item is <= item
#pragma unroll
  for (int step = 32; step > 0; step >>= 1)
    if (s_rex[own + step] <= item) own += step;
  const float4 uu = s_set[3 * own];
  const int r = static_cast<int>(item - s_rex[own]);
  if constexpr (kRect) {
    row = __float_as_int(uu.y) + r;
    tx0 = static_cast<uint32_t>(__float_as_int(uu.x));
    return static_cast<uint32_t>(__float_as_int(uu.z));
  } else {
    const float4 vv = s_set[3 * own + 1], ww = s_set[3 * own + 2];
    BandSetup bs;
    bs.mx = uu.x; bs.my = uu.y; bs.A = 0.0f; bs.B = uu.z; bs.det = uu.w;
    bs.tA = vv.x; bs.vmax = vv.y; bs.vr = vv.z; bs.invA = vv.w;
    bs.ok = bs.det > 0.0f;
    const int4 dd = make_int4(__float_as_int(ww.x), __float_as_int(ww.y), __float_as_int(ww.z), __float_as_int(ww.w));
    row = dd.z / kTile + r;
    int t0;
    const uint32_t nt = row_tiles(bs, dd, row, t0);
    tx0 = static_cast<uint32_t>(t0);
    return nt;
  }
}

// Spans as the row pass gathers them (depth order, one chunk's spans contiguous):
// x = Gaussian, y = tx0 | nt << 10 | row << 21 (tx0, row < 1024, nt <= 1024).
__device__ __forceinline__ uint32_t pack_row_span(uint32_t tx0, uint32_t nt, int row) {
  return tx0 | (nt << 10) | (static_cast<uint32_t>(row) << 21);
}

constexpr int kGatherHeld = 8;  // windows of (Gaussian, tile row) items a lane keeps between the passes

// Row pass, gather: one workgroup per chunk of kRowChunk Gaussians in depth order (wavefront w
// takes the w-th 64). Reads each Gaussian's record once, counts the chunk's non-empty spans per
// row into rowhist[r][c], reserves room for them in `gathered` (one atomic add per chunk:
// chunk_info[c] = (first slot, number of spans)) and writes them there in (Gaussian, row)
// order. The band arithmetic of the first kGatherHeld windows of items runs once (its spans are
// kept in registers between the passes), that of later windows twice (count, then write).
template <bool kRect>
__global__ __launch_bounds__(256) void span_gather_kernel(const SplatRec* __restrict__ rec,
                                                          const int4* __restrict__ rects,
                                                          const uint32_t* __restrict__ order, int64_t n,
                                                          int n_chunks, int tiles_x, int tiles_y,
                                                          uint32_t* __restrict__ rowhist,
                                                          uint2* __restrict__ chunk_info,
                                                          uint2* __restrict__ gathered, int64_t gathered_cap,
                                                          uint32_t* __restrict__ counter) {
  extern __shared__ __align__(16) uint32_t s_dyn[];
  __shared__ uint32_t s_wcnt[kSpanWaves];
  __shared__ uint32_t s_base;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // LDS: row counts [tiles_y]; per wavefront the band setups (3 float4), row prefix and ids of
  // its 64 Gaussians
  const int ty4 = align4i(tiles_y);
  uint32_t* s_cnt = s_dyn;
  uint32_t* s_wbase = s_dyn + ty4 + wave * (64 * 12 + 128);
  float4* s_set = reinterpret_cast<float4*>(s_wbase);
  uint32_t* s_rex = s_wbase + 64 * 12;
  uint32_t* s_gid = s_rex + 64;
  const int c = xcd_tile(blockIdx.x, gridDim.x);  // the grid has n_chunks workgroups
  for (int q = threadIdx.x; q < ty4; q += 256) s_cnt[q] = 0u;
  const int64_t j = static_cast<int64_t>(c) * kRowChunk + wave * kWave + lane;
  uint32_t rows = 0, g = 0;
  float4 u = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v = u, w = u;
  if (j < n) {
    g = order[j];
    if constexpr (kRect) {
      const int4 r = clamp_rect(rects[g], tiles_x, tiles_y);
      if (r.z > r.x && r.w > r.y) {
        rows = static_cast<uint32_t>(r.w - r.y);
        u = make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z - r.x), 0.0f);
      }
    } else {
      const float4 a = rec[g].a, b = rec[g].b;
      const int4 d = rec[g].d;
      if (d.w >= d.z && d.y >= d.x) {  // a culled record holds the empty bounds (0, -1, 0, -1)
        const BandSetup bs = band_setup(a, b);
        rows = static_cast<uint32_t>(d.w / kTile - d.z / kTile + 1);
        u = make_float4(bs.mx, bs.my, bs.B, bs.det);
        v = make_float4(bs.tA, bs.vmax, bs.vr, bs.invA);
        w = make_float4(__int_as_float(d.x), __int_as_float(d.y), __int_as_float(d.z), __int_as_float(d.w));
      }
    }
  }
  s_set[3 * lane] = u;
  s_set[3 * lane + 1] = v;
  s_set[3 * lane + 2] = w;
  s_gid[lane] = g;
  uint32_t total;
  s_rex[lane] = wave_excl_scan(rows, lane, total);
  __syncthreads();  // counts cleared, setups visible
  // the first kGatherHeld windows' spans are kept (packed, with their Gaussian's slot) for the
  // write pass; later windows are evaluated again there
  uint32_t held_pk[kGatherHeld], held_own[kGatherHeld];
  uint32_t live_total = 0;
#pragma unroll
  for (int u = 0; u < kGatherHeld; ++u) {
    held_pk[u] = 0u;
    held_own[u] = 0u;
    const uint32_t base = static_cast<uint32_t>(u * kWave);
    if (base >= total) continue;  // wave-uniform
    const uint32_t item = base + static_cast<uint32_t>(lane);
    bool live = false;
    if (item < total) {
      int own, row;
      uint32_t tx0;
      const uint32_t nt = row_item<kRect>(s_set, s_rex, item, own, row, tx0);
      live = nt > 0u;
      if (live) {
        atomicAdd(&s_cnt[row], 1u);
        held_pk[u] = pack_row_span(tx0, nt, row);  // nonzero: nt >= 1
        held_own[u] = static_cast<uint32_t>(own);
      }
    }
    live_total += static_cast<uint32_t>(__popcll(__ballot(live ? 1 : 0)));
  }
  for (uint32_t base = kGatherHeld * kWave; base < total; base += kWave) {
    const uint32_t item = base + static_cast<uint32_t>(lane);
    bool live = false;
    if (item < total) {
      int own, row;
      uint32_t tx0;
      live = row_item<kRect>(s_set, s_rex, item, own, row, tx0) > 0u;
      if (live) atomicAdd(&s_cnt[row], 1u);
    }
    live_total += static_cast<uint32_t>(__popcll(__ballot(live ? 1 : 0)));
  }
  if (lane == 0) s_wcnt[wave] = live_total;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t all = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
    const uint32_t first = all ? atomicAdd(counter, all) : 0u;
    s_base = first;
    chunk_info[c] = make_uint2(first, all);
  }
  for (int r = threadIdx.x; r < tiles_y; r += 256) rowhist[static_cast<int64_t>(r) * n_chunks + c] = s_cnt[r];
  __syncthreads();
  uint32_t slot = s_base;
  for (int q = 0; q < wave; ++q) slot += s_wcnt[q];
  const uint64_t lt = lanemask_lt(lane);
#pragma unroll
  for (int u = 0; u < kGatherHeld; ++u) {
    if (static_cast<uint32_t>(u * kWave) >= total) continue;  // wave-uniform
    const bool live = held_pk[u] != 0u;
    const uint64_t lv = __ballot(live ? 1 : 0);
    if (live) {
      const int64_t p = static_cast<int64_t>(slot) + __popcll(lv & lt);
      if (p < gathered_cap) gathered[p] = make_uint2(s_gid[held_own[u]], held_pk[u]);
    }
    slot += static_cast<uint32_t>(__popcll(lv));
  }
  for (uint32_t base = kGatherHeld * kWave; base < total; base += kWave) {
    const uint32_t item = base + static_cast<uint32_t>(lane);
    int own = 0, row = 0;
    uint32_t tx0 = 0, nt = 0;
    if (item < total) nt = row_item<kRect>(s_set, s_rex, item, own, row, tx0);
    const uint64_t lv = __ballot(nt > 0u ? 1 : 0);
    if (nt > 0u) {
      const int64_t p = static_cast<int64_t>(slot) + __popcll(lv & lt);
      if (p < gathered_cap) gathered[p] = make_uint2(s_gid[own], pack_row_span(tx0, nt, row));
    }
    slot += static_cast<uint32_t>(__popcll(lv));
  }
}

// Row pass, placement: one workgroup per chunk; its gathered spans, split into four contiguous
// quarters (one per wavefront), go to their rows: row start + the chunk's offset in the row
// (rowhist, scanned) + the earlier wavefronts' spans of that row + the span's rank among the
// wavefront's earlier spans of that row. Ranks inside a window of 64 spans come from a
// coverage mask per row (each span ORs its lane bit in; the rank is the number of lower bits).
// Writes (Gaussian, tx0 | nt << 16). A wavefront's first kPlaceHeld windows are loaded once,
// all loads issued together, and serve both the counting and the placement; longer quarters
// read the rest as they go.
constexpr int kPlaceHeld = 8;

// One window of up to 64 spans of a wavefront, in lane order (lane holds e when live).
__device__ __forceinline__ void place_window(bool live, uint2 e, int lane, uint64_t below, uint32_t* my_pos,
                                             unsigned long long* s_cov, uint2* __restrict__ spans,
                                             int64_t span_cap) {
  int row = 0;
  if (live) {
    row = static_cast<int>(e.y >> 21);
    atomicOr(&s_cov[row], 1ull << lane);
  }
  wave_sync();
  unsigned long long cov = 0ull;
  if (live) {
    cov = s_cov[row];
    const int64_t pos = static_cast<int64_t>(my_pos[row]) + __popcll(cov & below);
    if (pos < span_cap) spans[pos] = make_uint2(e.x, (e.y & 0x3ffu) | (((e.y >> 10) & 0x7ffu) << 16));
  }
  wave_sync();  // every lane has read its row's position and mask
  if (live && (cov & below) == 0ull) {  // the row's lowest lane advances it and clears the mask
    my_pos[row] += static_cast<uint32_t>(__popcll(cov));
    s_cov[row] = 0ull;
  }
  wave_sync();
}

__global__ __launch_bounds__(256) void span_place_kernel(const uint2* __restrict__ gathered,
                                                         const uint2* __restrict__ chunk_info,
                                                         const uint32_t* __restrict__ rowhist,
                                                         const uint32_t* __restrict__ rowtot, int n_chunks,
                                                         int tiles_y, uint2* __restrict__ spans,
                                                         int64_t gathered_cap, int64_t span_cap) {
  extern __shared__ __align__(16) uint32_t s_dyn[];
  __shared__ uint32_t s_wsum[kSpanWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // LDS: row bases [tiles_y + 1]; per wavefront: row positions [tiles_y], row coverage masks
  // [tiles_y] (uint64)
  const int ty4 = align4i(tiles_y);
  uint32_t* s_rbase = s_dyn;
  uint32_t* s_pos = s_dyn + align4i(tiles_y + 1);  // [kSpanWaves][ty4]
  unsigned long long* s_cov =
      reinterpret_cast<unsigned long long*>(s_pos + kSpanWaves * ty4) + static_cast<int64_t>(wave) * ty4;
  const int c = xcd_tile(blockIdx.x, gridDim.x);
  const uint2 info = chunk_info[c];
  const uint32_t q0 = static_cast<uint32_t>((static_cast<uint64_t>(info.y) * wave) / kSpanWaves);
  const uint32_t q1 = static_cast<uint32_t>((static_cast<uint64_t>(info.y) * (wave + 1)) / kSpanWaves);
  uint2 held[kPlaceHeld];
#pragma unroll
  for (int u = 0; u < kPlaceHeld; ++u) {
    const uint32_t i = q0 + static_cast<uint32_t>(u * kWave + lane);
    const int64_t p = static_cast<int64_t>(info.x) + i;
    held[u] = (i < q1 && p < gathered_cap) ? gathered[p] : make_uint2(0u, 0u);
  }
  span_row_bases<256>(rowtot, tiles_y, s_rbase, s_wsum);
  if (info.y == 0u) return;  // the whole workgroup: no spans
  uint32_t* my_pos = s_pos + wave * ty4;
  for (int q = threadIdx.x; q < kSpanWaves * ty4; q += 256) s_pos[q] = 0u;
  for (int q = lane; q < ty4; q += kWave) s_cov[q] = 0ull;
  __syncthreads();
  // count this quarter's spans per row
#pragma unroll
  for (int u = 0; u < kPlaceHeld; ++u) {
    const uint32_t i = q0 + static_cast<uint32_t>(u * kWave + lane);
    if (i < q1 && static_cast<int64_t>(info.x) + i < gathered_cap) atomicAdd(&my_pos[held[u].y >> 21], 1u);
  }
  for (uint32_t i = q0 + kPlaceHeld * kWave + lane; i < q1; i += kWave) {
    const int64_t p = static_cast<int64_t>(info.x) + i;
    if (p < gathered_cap) atomicAdd(&my_pos[gathered[p].y >> 21], 1u);
  }
  __syncthreads();
  for (int r = threadIdx.x; r < tiles_y; r += 256) {
    uint32_t run = s_rbase[r] + rowhist[static_cast<int64_t>(r) * n_chunks + c];
#pragma unroll
    for (int q = 0; q < kSpanWaves; ++q) {
      const uint32_t cnt = s_pos[q * ty4 + r];
      s_pos[q * ty4 + r] = run;
      run += cnt;
    }
  }
  __syncthreads();
  const uint64_t below = lanemask_lt(lane);
#pragma unroll
  for (int u = 0; u < kPlaceHeld; ++u) {
    const uint32_t i0 = q0 + static_cast<uint32_t>(u * kWave);
    if (i0 >= q1) break;  // wave-uniform
    const uint32_t i = i0 + static_cast<uint32_t>(lane);
    place_window(i < q1 && static_cast<int64_t>(info.x) + i < gathered_cap, held[u], lane, below, my_pos, s_cov,
                 spans, span_cap);
  }
  for (uint32_t i0 = q0 + kPlaceHeld * kWave; i0 < q1; i0 += kWave) {
    const uint32_t i = i0 + static_cast<uint32_t>(lane);
    const int64_t p = static_cast<int64_t>(info.x) + i;
    const bool live = i < q1 && p < gathered_cap;
    place_window(live, live ? gathered[p] : make_uint2(0u, 0u), lane, below, my_pos, s_cov, spans, span_cap);
  }
}

// Scan of the tile counts of a canvas (one workgroup of kBoThreads threads): ranges [start,
// end), bucket offsets (32 entries per bucket), optionally CSR tile offsets, and the bucket
// list header cleared.

__device__ void tile_scan_block(const uint32_t* __restrict__ cnt, int n_tiles, uint32_t* __restrict__ ranges,
                                uint32_t* __restrict__ boff, uint32_t* __restrict__ tile_offsets,
                                uint32_t* __restrict__ list_header) {
  __shared__ uint32_t s_wave[kBoThreads / kWave];
  __shared__ uint32_t s_wave_inst[kBoThreads / kWave];
  if (list_header && threadIdx.x < kListHeader) list_header[threadIdx.x] = 0u;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t run = 0, run_inst = 0;
  for (int c0 = 0; c0 < n_tiles; c0 += kBoThreads * kBoItems) {
    uint32_t len[kBoItems], sum = 0, sum_inst = 0;
#pragma unroll
    for (int e = 0; e < kBoItems; ++e) {
      const int t = c0 + static_cast<int>(threadIdx.x) * kBoItems + e;
      len[e] = t < n_tiles ? cnt[t] : 0u;
      sum += (len[e] + kBucket - 1) / kBucket;
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
        ranges[2 * t] = pos_inst;
        ranges[2 * t + 1] = pos_inst + len[e];
        if (tile_offsets) tile_offsets[t] = pos_inst;
      }
      pos += (len[e] + kBucket - 1) / kBucket;
      pos_inst += len[e];
    }
    run += total;
    run_inst += total_inst;
  }
  if (threadIdx.x == 0) {
    boff[n_tiles] = run;
    if (tile_offsets) tile_offsets[n_tiles] = run_inst;
  }
}

// Chunks of the column pass: chunk k (a workgroup) holds span positions [k kSpanChunk,
// (k + 1) kSpanChunk), all in one row (wavefront w takes the w-th kWaveSpans of them); row r's
// chunks are [cb, cb + nc) (clamped to the capacity). Chunk counts are stored chunk-major:
// colcnt[k][t] for column t.
constexpr int kWaveSpans = kSpanChunk / kSpanWaves;  // 256

struct SpanChunk {
  int row;
  int64_t cb, nc;  // the row's first chunk and its number of chunks
};

__device__ __forceinline__ SpanChunk span_chunk(const uint32_t* s_rbase, int tiles_y, int64_t k, int64_t chunk_cap) {
  SpanChunk sc;
  sc.row = span_row_of(s_rbase, tiles_y, static_cast<uint32_t>(k * kSpanChunk));
  sc.cb = min<int64_t>(s_rbase[sc.row] / kSpanChunk, chunk_cap);
  sc.nc = min<int64_t>(s_rbase[sc.row + 1] / kSpanChunk, chunk_cap) - sc.cb;
  return sc;
}

// The chunks of the column pass are dealt to the XCDs in contiguous ranges (a workgroup runs on
// XCD blockIdx.x % 8), so the chunks that write neighbouring parts of a tile's list share an
// L2. The grid is a multiple of 8 workgroups; workgroup `wid` of `nw` in its XCD takes chunks
// lo + wid, lo + wid + nw, ... below hi.
struct XcdRange {
  int64_t lo, hi, wid, nw;
};

__device__ __forceinline__ XcdRange xcd_range(int64_t n_items) {
  XcdRange x;
  const int xcd = static_cast<int>(blockIdx.x & 7u);
  x.lo = n_items * xcd / 8;
  x.hi = n_items * (xcd + 1) / 8;
  x.nw = static_cast<int64_t>(gridDim.x >> 3);
  x.wid = static_cast<int64_t>(blockIdx.x >> 3);
  return x;
}

// Instance counts per column of kWaveSpans spans (this wavefront's), from a difference array
// over the columns: s_cnt[t] for t < tiles_x (s_cnt holds tiles_x + 1 words). sp: the lane's
// kPerLane spans (empty ones have nt = 0).
constexpr int kPerLane = kWaveSpans / kWave;  // 4

__device__ __forceinline__ void wave_column_counts(const uint2 (&sp)[kPerLane], int tiles_x, int lane,
                                                   uint32_t* s_cnt) {
  for (int t = lane; t <= tiles_x; t += kWave) s_cnt[t] = 0u;
  wave_sync();
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) {
    const uint32_t tx0 = sp[e].y & 0xffffu, nt = sp[e].y >> 16;
    if (nt) {
      atomicAdd(&s_cnt[tx0], 1u);
      atomicAdd(&s_cnt[tx0 + nt], 0xffffffffu);
    }
  }
  wave_sync();
  const int per = (tiles_x + kWave - 1) / kWave;
  uint32_t sum = 0;
  for (int e = 0; e < per; ++e) {
    const int t = lane * per + e;
    if (t < tiles_x) sum += s_cnt[t];
  }
  uint32_t tot;
  uint32_t run = wave_excl_scan(sum, lane, tot);
  wave_sync();
  for (int e = 0; e < per; ++e) {
    const int t = lane * per + e;
    if (t < tiles_x) {
      run += s_cnt[t];
      s_cnt[t] = run;
    }
  }
  wave_sync();
}

// The lane's kPerLane consecutive spans of chunk k, wavefront `wave` (positions at or beyond lim
// are empty; a span reaching past the last column is dropped).
__device__ __forceinline__ void load_wave_spans(const uint2* __restrict__ spans, int64_t k, int wave, int lane,
                                                int64_t lim, int tiles_x, uint2 (&sp)[kPerLane]) {
  const int64_t p0 = k * kSpanChunk + wave * kWaveSpans + kPerLane * lane;
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) {
    sp[e] = p0 + e < lim ? spans[p0 + e] : make_uint2(0u, 0u);
    if ((sp[e].y & 0xffffu) + (sp[e].y >> 16) > static_cast<uint32_t>(tiles_x)) sp[e].y = 0u;
  }
}

// Column pass, counts: colcnt[k][t] = instances of chunk k in column t of its row.
__global__ __launch_bounds__(256) void span_col_count_kernel(const uint2* __restrict__ spans,
                                                             const uint32_t* __restrict__ rowtot, int tiles_x,
                                                             int tiles_y, int64_t span_cap, int64_t chunk_cap,
                                                             uint32_t* __restrict__ colcnt) {
  extern __shared__ __align__(16) uint32_t s_dyn[];
  __shared__ uint32_t s_wsum[kSpanWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tx4 = align4i(tiles_x + 1);
  uint32_t* s_rbase = s_dyn;
  uint32_t* s_cnt = s_dyn + align4i(tiles_y + 1);  // [kSpanWaves][tx4]
  span_row_bases<256>(rowtot, tiles_y, s_rbase, s_wsum);
  const int64_t n_chunks = min<int64_t>(s_rbase[tiles_y] / kSpanChunk, chunk_cap);
  const XcdRange xr = xcd_range(n_chunks);
  for (int64_t k = xr.lo + xr.wid; k < xr.hi; k += xr.nw) {
    const SpanChunk sc = span_chunk(s_rbase, tiles_y, k, chunk_cap);
    const int64_t lim = min<int64_t>(static_cast<int64_t>(s_rbase[sc.row]) + rowtot[sc.row], span_cap);
    uint2 sp[kPerLane];
    load_wave_spans(spans, k, wave, lane, lim, tiles_x, sp);
    wave_column_counts(sp, tiles_x, lane, s_cnt + wave * tx4);
    __syncthreads();
    for (int t = threadIdx.x; t < tiles_x; t += 256)
      colcnt[k * tiles_x + t] = s_cnt[t] + s_cnt[tx4 + t] + s_cnt[2 * tx4 + t] + s_cnt[3 * tx4 + t];
    __syncthreads();  // the counts are rewritten for the next chunk
  }
}

// Column pass, scan: workgroup r scans every column of row r over the row's chunks, in place
// (each chunk's offset within the tile), and writes the tile counts. The chunks are split into
// segments, a thread per (segment, column): segment sums, their prefix, then each thread
// rewrites its segment.
constexpr int kColScanMaxSegs = 32;

__global__ __launch_bounds__(kColScanThreads) void span_col_scan_kernel(uint32_t* __restrict__ colcnt,
                                                                        const uint32_t* __restrict__ rowtot,
                                                                        int tiles_x, int tiles_y, int64_t chunk_cap,
                                                                        uint32_t* __restrict__ tcnt) {
  __shared__ uint32_t s_rbase[kSpanMaxDim + 1];
  __shared__ uint32_t s_seg[kColScanThreads];
  __shared__ uint32_t s_wsum[kColScanThreads / kWave];
  span_row_bases<kColScanThreads>(rowtot, tiles_y, s_rbase, s_wsum);
  const int r = blockIdx.x;
  const int64_t cb = min<int64_t>(s_rbase[r] / kSpanChunk, chunk_cap);
  const int64_t ce = min<int64_t>(s_rbase[r + 1] / kSpanChunk, chunk_cap);
  int cols_p2 = 1;
  while (cols_p2 < tiles_x) cols_p2 <<= 1;
  const int segs = min(kColScanThreads / cols_p2, kColScanMaxSegs);
  const int col = static_cast<int>(threadIdx.x) & (cols_p2 - 1);
  const int seg = static_cast<int>(threadIdx.x) / cols_p2;
  const bool mine = col < tiles_x && seg < segs;
  const int64_t len = (ce - cb + segs - 1) / segs;
  const int64_t c0 = cb + seg * len;
  const int64_t c1 = min<int64_t>(c0 + len, ce);
  constexpr int kU = 8;  // loads in flight per thread
  uint32_t sum = 0;
  if (mine) {
    for (int64_t k = c0; k < c1; k += kU) {
      uint32_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = k + u < c1 ? colcnt[(k + u) * tiles_x + col] : 0u;
#pragma unroll
      for (int u = 0; u < kU; ++u) sum += v[u];
    }
  }
  s_seg[threadIdx.x] = mine ? sum : 0u;
  __syncthreads();
  if (!mine) return;  // no barrier follows
  uint32_t run = 0, total = 0;
  for (int s = 0; s < segs; ++s) {
    const uint32_t v = s_seg[s * cols_p2 + col];
    run += s < seg ? v : 0u;
    total += v;
  }
  for (int64_t k = c0; k < c1; k += kU) {
    uint32_t v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = k + u < c1 ? colcnt[(k + u) * tiles_x + col] : 0u;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (k + u < c1) colcnt[(k + u) * tiles_x + col] = run;
      run += v[u];
    }
  }
  if (seg == 0) tcnt[static_cast<int64_t>(r) * tiles_x + col] = total;
}

// Ranges, bucket offsets and the bucket list header from the tile counts (one workgroup).
__global__ __launch_bounds__(kBoThreads) void tile_scan_kernel(const uint32_t* __restrict__ tcnt, int n_tiles,
                                                              uint32_t* __restrict__ ranges,
                                                              uint32_t* __restrict__ boff,
                                                              uint32_t* __restrict__ tile_offsets,
                                                              uint32_t* __restrict__ list_header) {
  tile_scan_block(tcnt, n_tiles, ranges, boff, tile_offsets, list_header);
}

// Column pass, placement: workgroup per chunk, each wavefront places the instances of its
// kWaveSpans spans. Instance i of a wavefront's spans (numbered in (span, column) order) goes
// to its tile's start + the chunk's offset in the tile + the earlier wavefronts' instances in
// the column + its rank among the wavefront's earlier instances in the column. The instances
// are taken in batches of R windows of 64: an owner table gives each instance its span; in a
// window, each span (at most 64, all of distinct columns) ORs its bit (span - the window's first
// span) into the window's column mask, so the rank inside the window is the number of lower
// bits; a pass over the columns then turns the windows' counts into running positions.
constexpr int kOwnerTable = 2048;  // instances per owner-table segment (one byte each)

template <bool kKeys, int R>
__global__ __launch_bounds__(256) void span_col_write_kernel(
    const uint2* __restrict__ spans, const uint32_t* __restrict__ rowtot, const uint32_t* __restrict__ colcnt,
    const uint32_t* __restrict__ ranges, int tiles_x, int tiles_y, int64_t span_cap, int64_t chunk_cap, int64_t m,
    uint32_t* __restrict__ point_list, uint64_t* __restrict__ keys, const uint32_t* __restrict__ dkey_of,
    uint32_t dkey0) {
  extern __shared__ __align__(16) uint32_t s_dyn[];
  __shared__ uint32_t s_wsum[kSpanWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // LDS: row bases [tiles_y + 1]; column positions [kSpanWaves][tiles_x + 1]; per wavefront:
  // the windows' column masks [R][tiles_x] (uint64) and offsets [R][tiles_x], the spans
  // (uint2) and their instance prefix, the owner table (bytes)
  const int tx4 = align4i(tiles_x + 1);
  const int wave_words = R * 3 * tx4 + 2 * kWaveSpans + (kWaveSpans + 4) + kOwnerTable / 4;
  uint32_t* s_rbase = s_dyn;
  uint32_t* s_cpos = s_dyn + align4i(tiles_y + 1);  // [kSpanWaves][tx4]
  uint32_t* s_w = s_cpos + kSpanWaves * tx4 + wave * wave_words;
  unsigned long long* s_cov = reinterpret_cast<unsigned long long*>(s_w);  // [R][tx4]
  uint32_t* s_off = s_w + 2 * R * tx4;                                       // [R][tx4]
  uint2* s_span = reinterpret_cast<uint2*>(s_off + R * tx4);                 // [kWaveSpans]
  uint32_t* s_pre = s_off + R * tx4 + 2 * kWaveSpans;                        // [kWaveSpans + 1]
  uint8_t* s_tbl = reinterpret_cast<uint8_t*>(s_pre + kWaveSpans + 4);       // [kOwnerTable]
  uint32_t* s_pos = s_cpos + wave * tx4;
  span_row_bases<256>(rowtot, tiles_y, s_rbase, s_wsum);
  for (int q = lane; q < R * tx4; q += kWave) s_cov[q] = 0ull;
  const int64_t n_chunks = min<int64_t>(s_rbase[tiles_y] / kSpanChunk, chunk_cap);
  const XcdRange xr = xcd_range(n_chunks);
  for (int64_t k = xr.lo + xr.wid; k < xr.hi; k += xr.nw) {
    const SpanChunk sc = span_chunk(s_rbase, tiles_y, k, chunk_cap);
    const int64_t lim = min<int64_t>(static_cast<int64_t>(s_rbase[sc.row]) + rowtot[sc.row], span_cap);
    const int64_t t_row = static_cast<int64_t>(sc.row) * tiles_x;
    uint2 sp[kPerLane];
    load_wave_spans(spans, k, wave, lane, lim, tiles_x, sp);
    wave_column_counts(sp, tiles_x, lane, s_pos);
    __syncthreads();
    // each wavefront's first position in every column: the tile's start, the chunk's offset in
    // the tile, then the earlier wavefronts' instances
    for (int t = threadIdx.x; t < tiles_x; t += 256) {
      uint32_t run = ranges[2 * (t_row + t)] + colcnt[k * tiles_x + t];
#pragma unroll
      for (int q = 0; q < kSpanWaves; ++q) {
        const uint32_t c = s_cpos[q * tx4 + t];
        s_cpos[q * tx4 + t] = run;
        run += c;
      }
    }
    __syncthreads();
    // the wavefront's non-empty spans, compacted in order: span index c of s_span / s_pre is the
    // c-th non-empty one, so the 64 consecutive instances of a window always lie in at most 64
    // consecutive span indices (the rank bits below), whatever spans were empty
    uint32_t sum = 0, nz = 0;
#pragma unroll
    for (int e = 0; e < kPerLane; ++e) {
      sum += sp[e].y >> 16;
      nz += (sp[e].y >> 16) != 0u ? 1u : 0u;
    }
    uint32_t total, n_nz;
    uint32_t run = wave_excl_scan(sum, lane, total);
    uint32_t ci = wave_excl_scan(nz, lane, n_nz);
    uint32_t cidx[kPerLane];
#pragma unroll
    for (int e = 0; e < kPerLane; ++e) {
      cidx[e] = ci;
      if ((sp[e].y >> 16) != 0u) {
        s_pre[ci] = run;
        s_span[ci] = sp[e];
        ++ci;
      }
      run += sp[e].y >> 16;
    }
    uint32_t carry = 0u;  // the span holding the last instance of the previous segment
    for (uint32_t t0 = 0; t0 < total; t0 += kOwnerTable) {
      const uint32_t t1 = min<uint32_t>(t0 + kOwnerTable, total);
      wave_sync();  // the previous segment is done with the table
      // owner table: every instance of the segment gets its span's index. The spans' instances
      // are consecutive in span order, so the owner of instance i is the largest span index
      // whose first instance is at or before i: each non-empty span starting in the segment
      // marks its first entry, and a prefix maximum over the entries (seeded with the span
      // holding the segment's first instance) fills the rest, in the same few instructions
      // whatever the spans' widths.
      uint32_t* s_tw = reinterpret_cast<uint32_t*>(s_tbl);
      for (int q = lane; q < kOwnerTable / 4; q += kWave) s_tw[q] = 0u;
      wave_sync();
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) {
        if ((sp[e].y >> 16) == 0u) continue;
        const uint32_t st = s_pre[cidx[e]];
        if (st >= t0 && st < t1) s_tbl[st - t0] = static_cast<uint8_t>(cidx[e]);
      }
      wave_sync();
      {
        constexpr int kBytes = kOwnerTable / kWave;  // 32 consecutive entries per lane
        uint32_t w[kBytes / 4];
#pragma unroll
        for (int q = 0; q < kBytes / 4; ++q) w[q] = s_tw[lane * (kBytes / 4) + q];
        uint32_t run = 0u;
#pragma unroll
        for (int q = 0; q < kBytes / 4; ++q)
#pragma unroll
          for (int b = 0; b < 4; ++b) run = max(run, (w[q] >> (8 * b)) & 0xffu);
        // the largest marker of the lanes before this one (a wavefront max-scan), and the seed
        uint32_t incl = run;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
          const uint32_t u = __shfl_up(incl, o, 64);
          if (lane >= o) incl = max(incl, u);
        }
        uint32_t m = max(carry, __shfl_up(incl, 1, 64));
        if (lane == 0) m = carry;
#pragma unroll
        for (int q = 0; q < kBytes / 4; ++q) {
          uint32_t out = 0u;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            m = max(m, (w[q] >> (8 * b)) & 0xffu);
            out |= m << (8 * b);
          }
          s_tw[lane * (kBytes / 4) + q] = out;
        }
      }
      wave_sync();
      carry = s_tbl[t1 - 1 - t0];
      for (uint32_t b0 = t0; b0 < t1; b0 += R * kWave) {
        uint32_t col[R], g[R], bit[R], low[R];
        bool live[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t w0 = b0 + r * kWave;
          const uint32_t i = w0 + static_cast<uint32_t>(lane);
          live[r] = i < t1;
          col[r] = g[r] = bit[r] = 0u;
          if (live[r]) {
            const uint32_t own = s_tbl[i - t0];
            const uint32_t first = s_tbl[w0 - t0];  // the window's first span
            const uint2 e = s_span[own];
            col[r] = (e.y & 0xffffu) + (i - s_pre[own]);
            g[r] = e.x;
            bit[r] = own - first;  // < 64: 64 instances lie in at most 64 compacted spans
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (live[r]) atomicOr(&s_cov[r * tx4 + col[r]], 1ull << bit[r]);
        wave_sync();
#pragma unroll
        for (int r = 0; r < R; ++r)
          low[r] = live[r] ? static_cast<uint32_t>(__popcll(s_cov[r * tx4 + col[r]] & ((1ull << bit[r]) - 1ull))) : 0u;
        wave_sync();
        // the windows' counts per column -> running positions (and the masks cleared)
        for (int t = lane; t < tiles_x; t += kWave) {
          uint32_t p = s_pos[t];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            s_off[r * tx4 + t] = p;
            p += static_cast<uint32_t>(__popcll(s_cov[r * tx4 + t]));
            s_cov[r * tx4 + t] = 0ull;
          }
          s_pos[t] = p;
        }
        wave_sync();
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (live[r]) {
            const uint32_t pos = s_off[r * tx4 + col[r]] + low[r];
            if (pos < m) {
              point_list[pos] = g[r];
              if constexpr (kKeys)
                keys[pos] = (static_cast<uint64_t>(t_row + col[r]) << 32) |
                            static_cast<uint32_t>(dkey_of[g[r]] + dkey0);
            }
          }
        }
        wave_sync();  // the offsets are rewritten by the next batch
      }
    }
    __syncthreads();  // the column positions are rewritten for the next chunk
  }
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

// Span binning: row counts per depth chunk [tiles_y][n_chunks], row totals, the gathered
// spans (depth order; at most m non-empty ones) with each chunk's (first slot, count) and the
// slot counter, the row-sorted spans (plus each row's padding to a multiple of kSpanChunk),
// column counts per span chunk, tile counts.
static bool span_binning(int tiles_x, int tiles_y) { return tiles_x <= kSpanMaxDim && tiles_y <= kSpanMaxDim; }

// Which fill a canvas and Gaussian count take: the span binning on canvases of at most
// kSpanMaxDim tiles per side from kSpanMinGaussians Gaussians on (below that, the radix path was
// measured faster: 1M Gaussians at 1297x840 bin in 127 us by radix and 152 us by spans, 3M at
// 1957x1091 in 1.01 ms by radix and 0.81 ms by spans), unless flags force a path. The choice
// needs no instance count, so the depth ordering knows beforehand whether the fill needs the
// instance offsets.
constexpr int64_t kSpanMinGaussians = 2000000;

static bool use_spans(int64_t n, int tiles_x, int tiles_y, int flags) {
  if (!span_binning(tiles_x, tiles_y) || (flags & GS_BIN_RADIX)) return false;
  return (flags & GS_BIN_SPANS) || n >= kSpanMinGaussians;
}

// The 3D fill's path: the span binning as above; below it the instances are emitted in depth
// order and stably sorted by tile (GS_BIN_PATH_RADIX).
static int bin_path(int64_t n, int tiles_x, int tiles_y, int flags) {
  return use_spans(n, tiles_x, tiles_y, flags) ? GS_BIN_PATH_SPANS : GS_BIN_PATH_RADIX;
}

// m instances fit the span path's 32-bit span positions (m plus every row's padding)
static bool span_fits(int64_t m, int tiles_y) {
  return m + static_cast<int64_t>(tiles_y) * kSpanChunk < (int64_t(1) << 32);
}

struct SpanLayout {
  size_t rowhist, rowtot, gathered, chunk_info, counter, spans, colhist, tcnt, end;
  int n_chunks;
  int64_t gathered_cap, span_cap, chunk_cap;
};

static SpanLayout span_layout(int64_t n, int64_t m, int tiles_x, int tiles_y) {
  SpanLayout L;
  L.n_chunks = static_cast<int>((n + kRowChunk - 1) / kRowChunk);
  L.gathered_cap = m;
  L.span_cap = m + static_cast<int64_t>(tiles_y) * (kSpanChunk - 1);
  L.chunk_cap = (L.span_cap + kSpanChunk - 1) / kSpanChunk;
  size_t o = 0;
  L.rowhist = o; o += align_up(static_cast<size_t>(tiles_y) * L.n_chunks * 4);
  L.rowtot = o; o += align_up(static_cast<size_t>(tiles_y) * 4);
  L.gathered = o; o += align_up(static_cast<size_t>(L.gathered_cap) * 8);
  L.chunk_info = o; o += align_up(static_cast<size_t>(L.n_chunks) * 8);
  L.counter = o; o += align_up(4);
  L.spans = o; o += align_up(static_cast<size_t>(L.span_cap) * 8);
  L.colhist = o; o += align_up(static_cast<size_t>(L.chunk_cap) * tiles_x * 4);
  L.tcnt = o; o += align_up(static_cast<size_t>(tiles_x) * tiles_y * 4);
  L.end = o;
  return L;
}

// Workspace of the fill for n Gaussians and m instances: the span binning's or the emission's.
static size_t fill_ws(int64_t n, int64_t m, int tiles_x, int tiles_y, int flags) {
  if (bin_path(n, tiles_x, tiles_y, flags) == GS_BIN_PATH_SPANS) return span_layout(n, m, tiles_x, tiles_y).end;
  return emit_layout(m, tiles_x * tiles_y).end;
}

// Rectangle binning: the depth ordering, the order and offsets, then the fill.
struct RectLayout {
  size_t prep, order, offs, emit, end;
};

static RectLayout rect_layout(int64_t n, int64_t m, int tiles_x, int tiles_y, int flags) {
  RectLayout L;
  size_t o = 0;
  L.prep = o; o += prep_layout(n).end;
  L.order = o; o += align_up(n * 4);
  L.offs = o; o += align_up((n + 1) * 4);
  L.emit = o; o += fill_ws(n, m, tiles_x, tiles_y, flags);
  L.end = o;
  return L;
}

static size_t prep_ws(int64_t n) { return prep_layout(n).end; }

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
  stage_mark("start", st);
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
    stage_mark("depth_sort", st);
    if (offsets) {
      scan_rec(sorted_counts, offsets, n, scan_scratch, st);
      stage_mark("instance_offsets", st);
    }
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
    hipLaunchKernelGGL((emit_kernel<true, K>), dim3(grid_for(n_windows, kEmitWaves)), dim3(kEmitWaves * 64), 0, st, rec, rects, order,
                       offsets, n, wstart, n_windows, tiles_x, n_tiles / tiles_x, tkeys, tvals, preset, n_tiles);
  } else {
    hipLaunchKernelGGL((emit_kernel<false, K>), dim3(grid_for(n_windows, kEmitWaves)), dim3(kEmitWaves * 64), 0, st, rec, rects, order,
                       offsets, n, wstart, n_windows, tiles_x, n_tiles / tiles_x, tkeys, tvals, preset, n_tiles);
  }
  stage_mark("key_duplication", st);
  radix_sort(tkeys, tvals, tsorted, point_list, m, tile_bits, ws + L.sort, st, nullptr, nullptr, preset,
             preset != nullptr && !sorted_keys);
  stage_mark("tile_sort", st);
  if (sorted_keys)
    hipLaunchKernelGGL((full_keys_kernel<K>), dim3(grid_for(m, 256)), dim3(256), 0, st, tsorted, point_list, dkey_of,
                       dkey0, m, sorted_keys);
}

// Span binning of m > 0 instances (span_binning(tiles_x, tiles_y) holds): lists, ranges,
// bucket offsets, optional sorted keys (dkey_of needed then).
template <bool kRect>
static void bin_spans(const SplatRec* rec, const int4* rects, const uint32_t* dkey_of, uint32_t dkey0,
                      const uint32_t* order, int64_t n, int tiles_x, int tiles_y, int64_t m, uint64_t* sorted_keys,
                      uint32_t* point_list, uint32_t* ranges, uint32_t* tile_offsets, uint32_t* bucket_offsets,
                      uint32_t* list_header, char* ws, hipStream_t st) {
  const SpanLayout L = span_layout(n, m, tiles_x, tiles_y);
  uint32_t* rowhist = reinterpret_cast<uint32_t*>(ws + L.rowhist);
  uint32_t* rowtot = reinterpret_cast<uint32_t*>(ws + L.rowtot);
  uint2* gathered = reinterpret_cast<uint2*>(ws + L.gathered);
  uint2* chunk_info = reinterpret_cast<uint2*>(ws + L.chunk_info);
  uint32_t* counter = reinterpret_cast<uint32_t*>(ws + L.counter);
  uint2* spans = reinterpret_cast<uint2*>(ws + L.spans);
  uint32_t* colhist = reinterpret_cast<uint32_t*>(ws + L.colhist);
  uint32_t* tcnt = reinterpret_cast<uint32_t*>(ws + L.tcnt);
  const auto a4 = [](int v) { return (v + 3) & ~3; };
  // LDS of the kernels (the layouts the kernels carve, in words)
  const size_t lds_gather = static_cast<size_t>(a4(tiles_y) + kSpanWaves * (64 * 12 + 128)) * 4;
  const size_t lds_place = static_cast<size_t>(a4(tiles_y + 1) + kSpanWaves * a4(tiles_y) * 3) * 4;
  const int tx4 = a4(tiles_x + 1);
  const size_t lds_ccount = (static_cast<size_t>(a4(tiles_y + 1)) + kSpanWaves * tx4) * 4;
  // placement windows per batch: fewer windows cost more wavefront syncs per window, more cost LDS
  // and so occupancy; up to 128 tile columns the LDS stays near 36 KB (4 workgroups per CU)
  // (3M SH3, 123 columns: 351 us with 2 windows, 363 with 4, 379 with 1)
  const int R = tiles_x <= 64 ? 4 : tiles_x <= 256 ? 2 : 1;
  const size_t lds_cwrite =
      (static_cast<size_t>(a4(tiles_y + 1)) + kSpanWaves * tx4 +
       kSpanWaves * (R * 3 * tx4 + 2 * kWaveSpans + (kWaveSpans + 4) + kOwnerTable / 4)) * 4;
  const unsigned g_rows = static_cast<unsigned>(L.n_chunks);  // a workgroup per chunk
  // the column kernels deal their chunks to the 8 XCDs in contiguous ranges: a multiple of 8
  // workgroups
  const unsigned g_cols = std::min<unsigned>((static_cast<unsigned>(L.chunk_cap) + 7u) & ~7u, 2048u);
  hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, st, counter, int64_t(1), 0u);
  hipLaunchKernelGGL(span_gather_kernel<kRect>, dim3(g_rows), dim3(256), lds_gather, st, rec, rects, order, n,
                     L.n_chunks, tiles_x, tiles_y, rowhist, chunk_info, gathered, L.gathered_cap, counter);
  hipLaunchKernelGGL(rs_rowscan_kernel, dim3(tiles_y), dim3(kScanThreads), 0, st, rowhist, L.n_chunks, rowtot);
  hipLaunchKernelGGL(span_place_kernel, dim3(g_rows), dim3(256), lds_place, st, gathered, chunk_info, rowhist, rowtot,
                     L.n_chunks, tiles_y, spans, L.gathered_cap, L.span_cap);
  stage_mark("span_rows", st);
  hipLaunchKernelGGL(span_col_count_kernel, dim3(g_cols), dim3(256), lds_ccount, st, spans, rowtot, tiles_x, tiles_y,
                     L.span_cap, L.chunk_cap, colhist);
  hipLaunchKernelGGL(span_col_scan_kernel, dim3(tiles_y), dim3(kColScanThreads), 0, st, colhist, rowtot, tiles_x,
                     tiles_y, L.chunk_cap, tcnt);
  hipLaunchKernelGGL(tile_scan_kernel, dim3(1), dim3(kBoThreads), 0, st, tcnt, tiles_x * tiles_y, ranges,
                     bucket_offsets, tile_offsets, list_header);
  stage_mark("span_columns", st);
#define GS_SPAN_WRITE(KEYS, RR)                                                                                     \
  hipLaunchKernelGGL((span_col_write_kernel<KEYS, RR>), dim3(g_cols), dim3(256), lds_cwrite, st, spans, rowtot,     \
                     colhist, ranges, tiles_x, tiles_y, L.span_cap, L.chunk_cap, m, point_list, sorted_keys, dkey_of, \
                     dkey0)
  if (sorted_keys) {
    if (R == 4) GS_SPAN_WRITE(true, 4); else if (R == 2) GS_SPAN_WRITE(true, 2); else GS_SPAN_WRITE(true, 1);
  } else {
    if (R == 4) GS_SPAN_WRITE(false, 4); else if (R == 2) GS_SPAN_WRITE(false, 2); else GS_SPAN_WRITE(false, 1);
  }
#undef GS_SPAN_WRITE
  stage_mark("span_write", st);
}

static void bin_emit(const SplatRec* rec, const int4* rects, const uint32_t* dkey_of, uint32_t dkey0,
                     const uint32_t* order,
                     const uint32_t* offsets, int64_t n, int tiles_x, int tiles_y, int64_t m,
                     uint64_t* sorted_keys, uint32_t* point_list, uint32_t* ranges, uint32_t* tile_offsets,
                     uint32_t* bucket_offsets, uint32_t* list_header, int flags, char* ws, hipStream_t st) {
  const int n_tiles = tiles_x * tiles_y;
  stage_mark("start", st);
  if (m > 0 && use_spans(n, tiles_x, tiles_y, flags)) {
    // (gs_bin_fill_* reject an m beyond span_fits for this path)
    if (rects)
      bin_spans<true>(rec, rects, dkey_of, dkey0, order, n, tiles_x, tiles_y, m, sorted_keys, point_list, ranges,
                      tile_offsets, bucket_offsets, list_header, ws, st);
    else
      bin_spans<false>(rec, rects, dkey_of, dkey0, order, n, tiles_x, tiles_y, m, sorted_keys, point_list, ranges,
                       tile_offsets, bucket_offsets, list_header, ws, st);
    return;
  }
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
    const bool short_keys = sort_ranges && n_tiles <= 65536;
    if (short_keys)
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
    stage_mark("ranges_buckets", st);
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

namespace gs {
// The asynchronous count readback's per-thread, per-device resources (created on first use).
struct CountSide {
  hipStream_t side = nullptr;
  hipEvent_t after = nullptr, done = nullptr;
  unsigned long long* host_word = nullptr;  // pinned, coherent: the sum kernel stores to it directly
  bool pending = false;
};
constexpr int kCountMaxDevices = 64;
static thread_local CountSide g_count[kCountMaxDevices];
}  // namespace gs

extern "C" int gs_count_begin(const uint32_t* wave_counts, int64_t n_waves, int on_side_stream, void* stream) {
  clear_error();
  GS_REQUIRE(n_waves >= 0 && (n_waves == 0 || wave_counts), GS_ERR_ARG, "invalid count arguments");
  GS_REQUIRE(aligned(wave_counts, 4), GS_ERR_ALIGN, "wave_counts must be 4-byte aligned");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return check_launch("count_begin (device)");
  GS_REQUIRE(dev >= 0 && dev < kCountMaxDevices, GS_ERR_ARG, "device index %d out of range", dev);
  CountSide& c = g_count[dev];
  GS_REQUIRE(!c.pending, GS_ERR_ARG, "gs_count_begin: the previous count on this thread and device was not ended");
  if (!c.side) {
    if (hipStreamCreateWithFlags(&c.side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c.after, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c.done, hipEventDisableTiming) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&c.host_word), sizeof(unsigned long long), hipHostMallocCoherent) !=
            hipSuccess) {
      const int e = check_launch("count_begin (set-up)");
      c = CountSide{};  // (a partial set-up is retried on the next call; its pieces leak)
      return e ? e : GS_ERR_LAUNCH;
    }
  }
  hipStream_t st = as_stream(stream);
  hipStream_t run = st;
  if (on_side_stream) {
    if (hipEventRecord(c.after, st) != hipSuccess || hipStreamWaitEvent(c.side, c.after, 0) != hipSuccess)
      return check_launch("count_begin (event)");
    run = c.side;
  }
  // one thread stores the total straight into the pinned word: no copy to enqueue
  hipLaunchKernelGGL(sum_u32_kernel, dim3(1), dim3(kSumThreads), 0, run, wave_counts, n_waves, c.host_word);
  if (int e = check_launch("count_begin (sum)")) return e;
  if (hipEventRecord(c.done, run) != hipSuccess) return check_launch("count_begin (event)");
  c.pending = true;
  return GS_OK;
}

extern "C" int gs_count_end(uint64_t* m) {
  clear_error();
  GS_REQUIRE(m, GS_ERR_ARG, "null pointer argument");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return check_launch("count_end (device)");
  GS_REQUIRE(dev >= 0 && dev < kCountMaxDevices && g_count[dev].pending, GS_ERR_ARG,
             "gs_count_end without gs_count_begin on this thread and device");
  CountSide& c = g_count[dev];
  c.pending = false;
  if (hipEventSynchronize(c.done) != hipSuccess) return check_launch("count_end");
  *m = *c.host_word;
  return GS_OK;
}

extern "C" size_t gs_bin_prepare_workspace_size(int64_t n) { return prep_ws(n < 0 ? 0 : n); }

extern "C" int gs_bin_prepare_3d(const float* splat_rec, const uint32_t* tiles_touched,
                                 const uint32_t* depth_keys, int64_t n, const gs_camera* cam, uint32_t* order,
                                 uint32_t* offsets, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (int e = check_cam(cam)) return e;
  GS_REQUIRE(n >= 0 && n < (int64_t(1) << 32), GS_ERR_ARG, "invalid bin_prepare arguments");
  GS_REQUIRE(n == 0 || (order && (depth_keys || splat_rec) && (tiles_touched || (!offsets && depth_keys))),
             GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(aligned(splat_rec, 16), GS_ERR_ALIGN, "splat_rec must be 16-byte aligned");
  const size_t need = prep_ws(n);
  GS_REQUIRE(workspace_bytes >= need && workspace, GS_ERR_WORKSPACE,
             "bin_prepare workspace too small: need %zu bytes", need);
  bin_prepare(depth_keys ? nullptr : reinterpret_cast<const SplatRec*>(splat_rec), nullptr, nullptr, depth_keys,
              depth_key_bits(make_cam(*cam)), tiles_touched, n, order, offsets, static_cast<char*>(workspace),
              as_stream(stream));
  return check_launch("bin_prepare_3d");
}

extern "C" size_t gs_bin_workspace_size(int64_t n, int64_t m, int tiles_x, int tiles_y, int flags) {
  n = n < 0 ? 0 : n;
  tiles_x = tiles_x < 1 ? 1 : tiles_x;
  tiles_y = tiles_y < 1 ? 1 : tiles_y;
  m = m < 0 ? 0 : m;
  // the rectangle binning runs the depth ordering itself: its scratch, order and offsets too;
  // the 3D fill needs its own path's workspace
  return std::max(rect_layout(n, m, tiles_x, tiles_y, flags).end, fill_ws(n, m, tiles_x, tiles_y, flags));
}

extern "C" size_t gs_bin_fill_3d_workspace_size(int64_t n, int64_t m, const gs_camera* cam) {
  if (!cam || cam->width <= 0 || cam->height <= 0) return 0;
  const CamK k = make_cam(*cam);
  return fill_ws(n < 0 ? 0 : n, m < 0 ? 0 : m, k.tiles_x, k.tiles_y, cam->flags);
}

extern "C" int gs_bin_path(int64_t n, const gs_camera* cam) {
  if (!cam) return GS_BIN_PATH_RADIX;
  const CamK k = make_cam(*cam);
  return bin_path(n, k.tiles_x, k.tiles_y, cam->flags);
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
  const int path = bin_path(n, k.tiles_x, k.tiles_y, cam->flags);
  GS_REQUIRE(path != GS_BIN_PATH_SPANS || span_fits(m, k.tiles_y), GS_ERR_ARG,
             "%lld instances exceed the 32-bit span positions", static_cast<long long>(m));
  const size_t need = fill_ws(n, m, k.tiles_x, k.tiles_y, cam->flags);
  GS_REQUIRE(workspace_bytes >= need && workspace, GS_ERR_WORKSPACE,
             "binning workspace too small: need %zu bytes", need);
  GS_REQUIRE(m == 0 || (splat_rec && point_list), GS_ERR_ARG, "null pointer argument");
  GS_REQUIRE(m == 0 || order, GS_ERR_ARG, "the fill needs the order of gs_bin_prepare_3d");
  GS_REQUIRE(m == 0 || offsets || path == GS_BIN_PATH_SPANS, GS_ERR_ARG, "this fill emits instances: it needs the offsets");
  GS_REQUIRE(!(sorted_keys && m > 0 && !depth_keys), GS_ERR_ARG, "sorted_keys need depth_keys");
  GS_REQUIRE(aligned(splat_rec, 16), GS_ERR_ALIGN, "splat_rec must be 16-byte aligned");
  bin_emit(reinterpret_cast<const SplatRec*>(splat_rec), nullptr, depth_keys, k.dkey0, order,
           offsets, n, k.tiles_x,
           k.tiles_y, m, sorted_keys, point_list, ranges, nullptr, bucket_offsets, bucket_list, cam->flags,
           static_cast<char*>(workspace), as_stream(stream));
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
                                uint32_t* tile_offsets, uint32_t* bucket_offsets, uint32_t* order, int flags,
                                void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && m >= 0 && m < (int64_t(1) << 32) && tiles_x > 0 && tiles_y > 0, GS_ERR_ARG,
             "invalid sizes");
  GS_REQUIRE(static_cast<int64_t>(tiles_x) * tiles_y < kMaxTiles, GS_ERR_ARG, "too many tiles");
  GS_REQUIRE(depth_dtype == GS_FLOAT32 || depth_dtype == GS_FLOAT64, GS_ERR_ARG, "invalid depth dtype");
  GS_REQUIRE(ranges && bucket_offsets, GS_ERR_ARG, "null output");
  const bool spans = use_spans(n, tiles_x, tiles_y, flags);
  GS_REQUIRE(!spans || span_fits(m, tiles_y), GS_ERR_ARG, "%lld instances exceed the 32-bit span positions",
             static_cast<long long>(m));
  const size_t need = gs_bin_workspace_size(n, m, tiles_x, tiles_y, flags);
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
  const RectLayout L = rect_layout(n, m, tiles_x, tiles_y, flags);
  char* prep = ws + L.prep;
  uint32_t* dkeys = reinterpret_cast<uint32_t*>(prep + prep_layout(n).dkeys);
  uint32_t* ord = order ? order : reinterpret_cast<uint32_t*>(ws + L.order);
  uint32_t* offs = reinterpret_cast<uint32_t*>(ws + L.offs);
  if (n > 0 && (m > 0 || order)) {
    // the span binning reads the order only; the emission needs the instance offsets too
    const bool need_offs = m > 0 && !spans;
    bin_prepare(nullptr, d32, d64, nullptr, 32, counts, n, ord, need_offs ? offs : nullptr, prep, st);
    if (sorted_keys && m > 0 && !d32)  // index order: the depth part of the keys is 0
      hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, dkeys, n, 0u);
  }
  bin_emit(nullptr, reinterpret_cast<const int4*>(rects), dkeys, 0u, ord, offs, n, tiles_x, tiles_y, m, sorted_keys,
           point_list, ranges, tile_offsets, bucket_offsets, nullptr, flags, ws + L.emit, st);
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
