// Stable LSD radix sort of (key, uint32 value) pairs in 8-bit digits, shared by
// the CSR build (tgx_csr.hip) and the negative pool (tgx_negpool.hip).
//
// A pass is three steps over tiles of kTile keys:
//   hist    : per-tile digit counts, stored digit-major (count[d][tile]);
//   scan    : exclusive prefix of the counts (tile scans, recursively over
//             the tile sums), so count[d][tile] becomes the tile's first
//             output position for digit d;
//   scatter : the tile's keys in order, kThreads at a time; each wavefront
//             ranks equal digits among its lanes with eight ballots, the
//             workgroup adds the earlier wavefronts' and rounds' counts, and
//             every key lands at its stable position in an LDS copy of the
//             tile sorted by digit (the tile's digit counts are differences of
//             the scanned counts); then the copy goes out in order, so the
//             keys of one digit leave as a run of consecutive positions
//             instead of one scattered store each (C3's first node pass:
//             216 -> 132 us for 20M keys).
// Everything lives in an anonymous namespace: each including file gets its own
// copy of the kernels.
#pragma once

#include "tgx_internal.h"

#include <algorithm>
#include <type_traits>
#include <vector>

namespace tgx {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kItems = 8;                 // keys per thread per tile
constexpr int kTile = kThreads * kItems;  // keys per tile (and scan tile)
constexpr int kBins = 256;                // 8-bit digits
static_assert(kBins == kThreads, "one digit per thread in the prefix step");

template <typename K>
__device__ __forceinline__ int digit_of(K k, int shift) {
  return static_cast<int>((k >> shift) & (kBins - 1));
}

template <typename K>
__global__ __launch_bounds__(kThreads) void radix_hist(const K* __restrict__ keys, int64_t n,
                                                       int shift, int64_t ntiles,
                                                       uint32_t* __restrict__ count) {
  __shared__ uint32_t h[kBins];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const int64_t j = base + r * kThreads + threadIdx.x;
    if (j < n) atomicAdd(&h[digit_of(keys[j], shift)], 1u);
  }
  __syncthreads();
  count[static_cast<int64_t>(threadIdx.x) * ntiles + blockIdx.x] = h[threadIdx.x];
}

// exclusive scan of data[tile * kTile, +kTile) in place; the tile total goes
// to sums[tile]
__global__ __launch_bounds__(kThreads) void scan_tiles(uint32_t* __restrict__ data, int64_t L,
                                                       uint32_t* __restrict__ sums) {
  __shared__ uint32_t wtot[kWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile + static_cast<int64_t>(threadIdx.x) * kItems;
  uint32_t v[kItems];
  uint32_t s = 0;
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    v[r] = base + r < L ? data[base + r] : 0u;
    s += v[r];
  }
  uint32_t incl = s;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += y;
  }
  if (lane == kWave - 1) wtot[wv] = incl;
  __syncthreads();
  uint32_t before = 0, total = 0;
  for (int w = 0; w < kWaves; ++w) {
    if (w < wv) before += wtot[w];
    total += wtot[w];
  }
  uint32_t run = before + incl - s;
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    if (base + r < L) data[base + r] = run;
    run += v[r];
  }
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(kThreads) void scan_add(uint32_t* __restrict__ data, int64_t L,
                                                     const uint32_t* __restrict__ sums) {
  const uint32_t add = sums[blockIdx.x];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const int64_t j = base + r * kThreads + threadIdx.x;
    if (j < L) data[j] += add;
  }
}

template <typename K>
__global__ __launch_bounds__(kThreads) void radix_scatter(const K* __restrict__ kin,
                                                          const uint32_t* __restrict__ vin,
                                                          K* __restrict__ kout,
                                                          uint32_t* __restrict__ vout, int64_t n,
                                                          int shift, int64_t ntiles,
                                                          const uint32_t* __restrict__ count) {
  __shared__ uint32_t gbase[kBins];          // first output position of the tile's digit d
  __shared__ uint32_t lstart[kBins];         // first local position of digit d
  __shared__ uint32_t lnext[kBins];          // next local position per digit
  __shared__ uint32_t wcnt[kWaves][kBins];   // this round's count per wave and digit
  __shared__ uint32_t wpos[kWaves][kBins];   // this round's first position per wave and digit
  __shared__ uint32_t wtot[kWaves];
  __shared__ K skey[kTile];                  // the tile in digit order
  __shared__ uint32_t sval[kTile];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  {  // digit threadIdx.x: its output start and, from the next scanned count, its
     // number of keys in this tile; their exclusive prefix is the local start
    const int64_t L = static_cast<int64_t>(kBins) * ntiles;
    const int64_t i = static_cast<int64_t>(threadIdx.x) * ntiles + blockIdx.x;
    const uint32_t g0 = count[i];
    const uint32_t c = (i + 1 < L ? count[i + 1] : static_cast<uint32_t>(n)) - g0;
    uint32_t incl = c;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t y = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += y;
    }
    if (lane == kWave - 1) wtot[wv] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wv; ++w) before += wtot[w];
    gbase[threadIdx.x] = g0;
    lstart[threadIdx.x] = before + incl - c;
    lnext[threadIdx.x] = before + incl - c;
  }
  for (int r = 0; r < kItems; ++r) {
    const int64_t j = base + r * kThreads + threadIdx.x;
    const bool valid = j < n;
    const K k = valid ? kin[j] : K(0);
    const uint32_t v = valid ? (vin != nullptr ? vin[j] : static_cast<uint32_t>(j)) : 0u;  // NULL: the identity
    const int d = digit_of(k, shift);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wcnt[w][threadIdx.x] = 0;
    __syncthreads();
    // lanes with the same digit: AND of the eight bit ballots
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool on = (d >> bit) & 1;
      const uint64_t m = __ballot(on);
      peers &= on ? m : ~m;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lt));
    if (valid && rank == 0) wcnt[wv][d] = static_cast<uint32_t>(__popcll(peers));
    __syncthreads();
    {  // digit threadIdx.x: local positions of the waves in order, then advance
      const int dd = threadIdx.x;
      uint32_t p = lnext[dd];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        wpos[w][dd] = p;
        p += wcnt[w][dd];
      }
      lnext[dd] = p;
    }
    __syncthreads();
    if (valid) {
      const uint32_t at = wpos[wv][d] + rank;
      skey[at] = k;
      sval[at] = v;
    }
  }
  __syncthreads();
  // the tile in digit order: runs of one digit go out to consecutive positions
  const int tn = static_cast<int>(n - base < kTile ? n - base : kTile);
  for (int i = threadIdx.x; i < tn; i += kThreads) {
    const K k = skey[i];
    const int d = digit_of(k, shift);
    const uint32_t at = gbase[d] + (static_cast<uint32_t>(i) - lstart[d]);
    kout[at] = k;
    vout[at] = sval[i];
  }
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// scan levels: L counts, then the tile sums of each level until one tile is left
std::vector<int64_t> scan_levels(int64_t L) {
  std::vector<int64_t> lv;
  int64_t m = L;
  while (true) {
    const int64_t t = cdiv(m, kTile);
    lv.push_back(t);
    if (t <= 1) break;
    m = t;
  }
  return lv;
}

// exclusive scan of data[0, L) with the tile-sum levels at `sums`
int scan_exclusive(uint32_t* data, int64_t L, uint32_t* sums, const std::vector<int64_t>& levels,
                   size_t level, hipStream_t stream) {
  const int64_t t = levels[level];
  hipLaunchKernelGGL(scan_tiles, dim3(static_cast<unsigned>(t)), dim3(kThreads), 0, stream, data, L, sums);
  int rc = check_launch("scan_tiles");
  if (rc || t <= 1) return rc;
  if ((rc = scan_exclusive(sums, t, sums + t, levels, level + 1, stream))) return rc;
  hipLaunchKernelGGL(scan_add, dim3(static_cast<unsigned>(t)), dim3(kThreads), 0, stream, data, L,
                     static_cast<const uint32_t*>(sums));
  return check_launch("scan_add");
}

struct RadixScratch;

template <typename K>
int radix_pass(const K* kin, const uint32_t* vin, K* kout, uint32_t* vout, int64_t n, int shift,
               const RadixScratch& w, uint32_t* count, uint32_t* sums, hipStream_t stream);

template <typename K>
int radix_pass_impl(const K* kin, const uint32_t* vin, K* kout, uint32_t* vout, int64_t n, int shift,
                    int64_t ntiles, const std::vector<int64_t>& levels, uint32_t* count, uint32_t* sums,
                    hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ntiles));
  hipLaunchKernelGGL(radix_hist<K>, grid, dim3(kThreads), 0, stream, kin, n, shift, ntiles, count);
  int rc = check_launch("radix_hist");
  if (rc) return rc;
  if ((rc = scan_exclusive(count, static_cast<int64_t>(kBins) * ntiles, sums, levels, 0, stream)))
    return rc;
  hipLaunchKernelGGL(radix_scatter<K>, grid, dim3(kThreads), 0, stream, kin, vin, kout, vout, n, shift,
                     ntiles, static_cast<const uint32_t*>(count));
  return check_launch("radix_scatter");
}


// counts and scan sums of a sort of n keys
struct RadixScratch {
  int64_t ntiles = 0;
  std::vector<int64_t> levels;
  size_t count_bytes = 0, sums_bytes = 0;
};

RadixScratch radix_scratch(int64_t n) {
  RadixScratch r;
  r.ntiles = std::max<int64_t>(cdiv(n, kTile), 1);
  const int64_t L = static_cast<int64_t>(kBins) * r.ntiles;
  r.levels = scan_levels(L);
  size_t nsums = 0;
  for (int64_t t : r.levels) nsums += static_cast<size_t>(t);
  r.count_bytes = align256(static_cast<size_t>(L) * 4);
  r.sums_bytes = align256(nsums * 4 + 4);
  return r;
}

template <typename K>
int radix_pass(const K* kin, const uint32_t* vin, K* kout, uint32_t* vout, int64_t n, int shift,
               const RadixScratch& w, uint32_t* count, uint32_t* sums, hipStream_t stream) {
  return radix_pass_impl<K>(kin, vin, kout, vout, n, shift, w.ntiles, w.levels, count, sums, stream);
}

// passes over bits [0, bits) of the keys, ping-ponging between k[0]/v[0] and
// k[1]/v[1]; `cur` is the buffer holding the input, and then the output.  With
// ident_values the first pass takes the values 0, 1, ..., n-1 without reading them
template <typename K>
int radix_sort(K* k[2], uint32_t* v[2], int& cur, int64_t n, int bits, const RadixScratch& r,
               uint32_t* count, uint32_t* sums, hipStream_t stream, bool ident_values = false) {
  for (int shift = 0; shift < bits; shift += 8) {
    const uint32_t* vin = shift == 0 && ident_values ? nullptr : v[cur];
    const int rc = radix_pass<K>(k[cur], vin, k[1 - cur], v[1 - cur], n, shift, r, count, sums, stream);
    if (rc) return rc;
    cur = 1 - cur;
  }
  return TGX_OK;
}

}  // namespace
}  // namespace tgx
