// Historical negative pool (reference pipeline/negatives.py:14-126): per node a
// pool of P destination ids kept by reservoir sampling over every edge seen
// from that node, and uniform draws from it.
//
// update(src, dst): edge j of the batch, the r-th of its source u in batch
// order, is u's e-th edge overall, e = count[u] + r + 1.  While e <= P it fills
// slot e-1; after that it replaces a random slot with probability P/e
// (float32, as the reference computes it).  The reference resolves two
// accepted edges on one (u, slot) by whichever index_put_ write lands last;
// here the later edge of the batch wins.  count[u] += (edges of u).
//
// With the caller's cell table (scratch), batches of up to 32,768 edges: two
// launches over the device (np_rank, np_commit below): ordered ranks from an LDS
// hash of each workgroup's sources and one scan of the batch, the decisions, and
// the latest edge per cell u*P + slot by atomicMax in the table.
// Otherwise, batches of more than 8,192 edges (several launches):
//   1. stable radix sort of the edges by source (tgx_radix.h): r = position
//      - start of the source's run;
//   2. decide: fill / replace / skip, and the key u*P + slot of accepted edges;
//   3. stable radix sort of accepted edges by that key: the last of each equal
//      run is the latest edge, which writes the slot;
//   4. counts: the last edge of each source run adds the run length.
// and batches of up to 8,192 edges: the same steps in one workgroup
// (np_update_small below), grouping sources through LDS hash tables.
//
// sample(src): with v = min(count[u], P) valid slots (slots fill in order, so
// they are a prefix), slot = int(f32(U) * f32(v)) clamped to P-1, else a
// random node when u has no history.
//
// Random numbers: rand64(seed, call, i, stream) = mix(mix(mix(seed ^ G) ^ call)
// ^ (4 i + stream)) with mix the splitmix64 finalizer and G its golden-ratio
// increment; U = (rand64 >> 40) * 2^-24.  Streams: 0 accept, 1 replacement
// slot (update); 2 slot, 3 fallback node (sample).
//
// Caller draws (tgx_negpool_update_draws / tgx_negpool_sample_draws): the
// uniforms and replacement slots come from the caller, indexed as the
// reference indexes its torch.rand / torch.randint draws -- by the edge's
// position in the stable sort of the batch by source (update), by query
// (sample) -- so a caller drawing them from torch's generator in the
// reference's order reproduces its pool and samples.  The update then takes
// the sort-based path (positions by node id); a sample of a source without
// history is left to the caller (-1), which draws its node afterwards as the
// reference does.
#include "tgx_radix.h"
#include "tgx_ring_plan.h"

#include <mutex>

namespace tgx {
namespace {

constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ull;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rand64(uint64_t seed, uint64_t call, uint64_t i, uint64_t stream) {
  return mix64(mix64(mix64(seed ^ kGolden) ^ call) ^ (4 * i + stream));
}

__device__ __forceinline__ float uniform01(uint64_t h) {
  return static_cast<float>(h >> 40) * 5.9604644775390625e-08f;  // 2^-24
}

constexpr uint32_t kBadKey = 0xffffffffu;
constexpr uint64_t kSkip = ~uint64_t(0);

__global__ __launch_bounds__(kThreads) void np_keys(const int64_t* __restrict__ src, int64_t n, int64_t N,
                                                    uint32_t* __restrict__ key, uint32_t* __restrict__ idx,
                                                    int32_t* __restrict__ status) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  bool bad = false;
  if (j < n) {
    const int64_t u = src[j];
    bad = u < 0 || u >= N;
    key[j] = bad ? kBadKey : static_cast<uint32_t>(u);
    idx[j] = static_cast<uint32_t>(j);
  }
  const uint64_t bm = __ballot(bad);
  if ((threadIdx.x & (kWave - 1)) == 0 && bm != 0 && status != nullptr)
    atomicAdd(&status[TGX_ST_BAD_EVENT_NODE], __popcll(bm));
}

// start of the run of key k in the sorted keys
__device__ __forceinline__ int64_t run_start(const uint32_t* __restrict__ skey, int64_t n, uint32_t k) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (skey[mid] < k)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kThreads) void np_decide(const uint32_t* __restrict__ skey,
                                                      const uint32_t* __restrict__ sidx, int64_t n,
                                                      const int64_t* __restrict__ count, int P,
                                                      uint64_t seed, uint64_t call,
                                                      const float* __restrict__ u_accept,
                                                      const int64_t* __restrict__ slot_draw,
                                                      uint64_t* __restrict__ ckey,
                                                      uint32_t* __restrict__ cval) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (p >= n) return;
  const uint32_t u = skey[p];
  const uint32_t j = sidx[p];
  uint64_t key = kSkip;
  if (u != kBadKey) {
    const int64_t r = p - run_start(skey, n, u);
    const int64_t e = count[u] + r + 1;
    int64_t slot = -1;
    if (e <= P) {
      slot = e - 1;
    } else if (u_accept != nullptr) {
      // the caller's draws of sorted position p; a slot outside [0, P) is skipped
      if (u_accept[p] < static_cast<float>(P) / static_cast<float>(e)) {
        slot = slot_draw[p];
        if (slot < 0 || slot >= P) slot = -1;
      }
    } else if (uniform01(rand64(seed, call, j, 0)) < static_cast<float>(P) / static_cast<float>(e)) {
      slot = static_cast<int64_t>(rand64(seed, call, j, 1) % static_cast<uint64_t>(P));
    }
    if (slot >= 0) key = static_cast<uint64_t>(u) * static_cast<uint64_t>(P) + static_cast<uint64_t>(slot);
  }
  ckey[p] = key;
  cval[p] = j;
}

__global__ __launch_bounds__(kThreads) void np_write(const uint64_t* __restrict__ ckey,
                                                     const uint32_t* __restrict__ cval, int64_t n,
                                                     const int64_t* __restrict__ dst,
                                                     int32_t* __restrict__ pool) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (q >= n) return;
  const uint64_t k = ckey[q];
  if (k == kSkip) return;
  if (q + 1 < n && ckey[q + 1] == k) return;  // a later edge takes this slot
  pool[k] = static_cast<int32_t>(dst[cval[q]]);
}

__global__ __launch_bounds__(kThreads) void np_count(const uint32_t* __restrict__ skey, int64_t n,
                                                     int64_t* __restrict__ count) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (p >= n) return;
  const uint32_t u = skey[p];
  if (u == kBadKey || (p + 1 < n && skey[p + 1] == u)) return;
  count[u] += p - run_start(skey, n, u) + 1;
}

__global__ __launch_bounds__(kThreads) void np_sample(const int32_t* __restrict__ pool,
                                                      const int64_t* __restrict__ count, int64_t N, int P,
                                                      const int64_t* __restrict__ src, int64_t n,
                                                      uint64_t seed, uint64_t call,
                                                      const float* __restrict__ u_slot,
                                                      int64_t* __restrict__ out,
                                                      int32_t* __restrict__ status) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  bool bad = false;
  if (q < n) {
    const int64_t u = src[q];
    bad = u < 0 || u >= N;
    const int64_t c = bad ? 0 : count[u];
    const int64_t v = c < P ? c : P;
    if (v > 0) {
      const float U = u_slot != nullptr ? u_slot[q] : uniform01(rand64(seed, call, q, 2));
      int64_t s = static_cast<int64_t>(U * static_cast<float>(v));
      if (s > P - 1) s = P - 1;
      out[q] = pool[u * P + s];
    } else {
      out[q] = u_slot != nullptr ? -1 : static_cast<int64_t>(rand64(seed, call, q, 3) % static_cast<uint64_t>(N));
    }
  }
  const uint64_t bm = __ballot(bad);
  if ((threadIdx.x & (kWave - 1)) == 0 && bm != 0 && status != nullptr)
    atomicAdd(&status[TGX_ST_BAD_QUERY_NODE], __popcll(bm));
}

// Batches of up to kNpRankMax edges with the caller's cell table (scratch): two
// launches over the whole device.
//   np_rank   : each workgroup ranks its edges among their source's edges in
//               batch order (rank_block of tgx_ring_plan.h: an LDS hash of its
//               sources and one scan of the batch's sources), so edge j, the
//               r-th of the c edges of u, decides as above with e = count[u] +
//               r + 1; an accepted edge finds its cell u * P + slot in the
//               table (open addressing on the key + 1, 0 = empty) and raises
//               the cell's latest edge to j + 1 (atomicMax).  The record of
//               edge j: (its cell or -1, the new count on u's last edge or -1).
//   np_commit : the cell's latest edge writes the pool slot and empties the
//               cell (the table is zero again after every call); u's last edge
//               writes count[u].  An edge that reads the cell after its latest
//               edge emptied it sees 0, which is not its own index either.
constexpr int64_t kNpRankMax = 32768;  // rank_block's before/after counts (< 2^15)
constexpr int kNpCellBits = 16;        // 65,536 cells: at most half full at kNpRankMax edges
constexpr int64_t kNpCells = int64_t(1) << kNpCellBits;

struct NpRankParams {
  const int64_t* src;
  int64_t n;
  int64_t N;
  int P;
  const int64_t* count;
  uint64_t seed;
  uint64_t call;
  unsigned long long* ckey;  // [kNpCells] cell + 1, 0 = empty
  int32_t* cmax;             // [kNpCells] latest edge + 1, 0 = none
  longlong2* rec;            // [n]
  int32_t* status;
};

__device__ __forceinline__ uint32_t np_cell_hash(uint64_t k) {
  return static_cast<uint32_t>((k * kGolden) >> (64 - kNpCellBits));
}

template <int T, int SCAN>
__global__ __launch_bounds__(T) void np_rank(NpRankParams P) {
  __shared__ __align__(16) uint8_t smem[plan_lds_bytes(T)];
  const int bad = rank_block<SCAN>(P.src, P.src, P.n, P.n, P.N, P.count, blockIdx.x, smem,
                                   [&](int64_t j, int32_t u, int c, int r, int64_t cnt) {
    int64_t cell = -1, newc = -1;
    if (u >= 0) {
      const int64_t e = cnt + r + 1;
      int64_t slot = -1;
      if (e <= P.P) {
        slot = e - 1;
      } else if (uniform01(rand64(P.seed, P.call, j, 0)) < static_cast<float>(P.P) / static_cast<float>(e)) {
        slot = static_cast<int64_t>(rand64(P.seed, P.call, j, 1) % static_cast<uint64_t>(P.P));
      }
      if (slot >= 0) {
        const uint64_t k1 = static_cast<uint64_t>(u) * static_cast<uint64_t>(P.P) + static_cast<uint64_t>(slot) + 1u;
        uint32_t h = np_cell_hash(k1);
        while (true) {  // terminates: at most n < kNpCells cells are ever taken
          const unsigned long long old = atomicCAS(&P.ckey[h], 0ull, static_cast<unsigned long long>(k1));
          if (old == 0ull || old == k1) break;
          h = (h + 1u) & static_cast<uint32_t>(kNpCells - 1);
        }
        atomicMax(&P.cmax[h], static_cast<int32_t>(j + 1));
        cell = h;
      }
      if (r == c - 1) newc = cnt + c;
    }
    P.rec[j] = make_longlong2(cell, newc);
  });
  const uint64_t bm = __ballot(bad);
  if ((threadIdx.x & (kWave - 1)) == 0 && bm != 0 && P.status != nullptr)
    atomicAdd(&P.status[TGX_ST_BAD_EVENT_NODE], __popcll(bm));
}

__global__ __launch_bounds__(kThreads) void np_commit(const longlong2* __restrict__ rec,
                                                      const int64_t* __restrict__ src,
                                                      const int64_t* __restrict__ dst, int64_t n,
                                                      unsigned long long* ckey, int32_t* cmax,
                                                      int32_t* __restrict__ pool, int64_t* __restrict__ count) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (j >= n) return;
  const longlong2 r = rec[j];
  const int64_t v = dst[j];
  const int64_t u = src[j];
  if (r.x >= 0) {
    const int32_t m = cmax[r.x];
    const unsigned long long k1 = ckey[r.x];
    if (m == static_cast<int32_t>(j + 1)) {
      pool[k1 - 1u] = static_cast<int32_t>(v);
      ckey[r.x] = 0ull;
      cmax[r.x] = 0;
    }
  }
  if (r.y >= 0) count[u] = r.y;
}

// Batches of at most 8,192 edges: the whole update in one workgroup (the
// sort-based path above costs some 25 launches, which a small batch cannot
// amortise).  Edge j is element j, held by thread j % 1024 in round j / 1024.
//
//   1. every source gets a slot of an LDS hash table (open addressing, twice as
//      many slots as edges); an out-of-range source gets the key after the slots;
//   2. a stable LSD radix sort of the words key << IBITS | j by the key, in PASSES
//      passes of DBITS bits: per round a wavefront ranks its 64 elements by digit
//      with ballots, the (digit, round, wavefront) counts are scanned in that
//      order, and each element lands at its offset plus its rank -- so a
//      source's edges end up together, in batch order;
//   3. rank r = position - first position of the key, the decision as on the
//      sort-based path, and the count added at the last position of each key;
//   4. accepted edges meet in a second LDS hash table on their cell u * P + slot,
//      whose entry keeps the largest cell << IBITS | j (atomicMax): that edge, the
//      batch's latest on the cell, writes it.
constexpr int kNpSmallThreads = 1024;
constexpr int kNpWaves = kNpSmallThreads / kWave;
constexpr int kNpEmpty = -1;
constexpr uint64_t kNpNone = ~uint64_t(0);

template <int CAP, int DBITS, int PASSES>
struct NpShape {
  static constexpr int kPer = CAP / kNpSmallThreads;  // rounds (elements per thread)
  static constexpr int kIBits = CAP == 4096 ? 12 : 13;  // edge index bits
  static constexpr int kSlots = 2 * CAP;                // hash slots of both tables
  static constexpr int kSlotBits = kIBits + 1;
  static constexpr int kBadKey = kSlots;                // sorts after every slot
  static constexpr int kDigits = 1 << DBITS;
  static constexpr int kTable = kDigits * kPer * kNpWaves;  // (digit, round, wavefront) counts
  // LDS: the source table (int32) and the sort's two element arrays (uint32) share
  // the bytes of the later cell table (uint64); the count table follows
  static constexpr size_t kLdsSort = static_cast<size_t>(kSlots) * 4;
  static constexpr size_t kLdsTable = static_cast<size_t>(kSlots) * 8;
  static constexpr size_t kLds = kLdsTable + static_cast<size_t>(kTable) * 4;
  static_assert((1 << kIBits) == CAP, "edge indices fill their bits");
  static_assert(kBadKey < (1 << (DBITS * PASSES)), "the passes cover the key");
  static_assert(kSlotBits + 1 + kIBits <= 32, "a sort word is 32 bits");
  static_assert(kTable % kNpSmallThreads == 0, "the scan takes whole runs per thread");
  static_assert(kLdsSort + 2 * static_cast<size_t>(CAP) * 4 <= kLdsTable, "the sort arrays end before the count table");
  static_assert(kLds <= 160 * 1024, "the workgroup's LDS");
};
using NpSmall = NpShape<4096, 7, 2>;
using NpMid = NpShape<8192, 5, 3>;

template <class S>
__device__ __forceinline__ uint32_t np_hash32(uint32_t u) {
  return (u * 2654435761u) >> (32 - S::kSlotBits);
}
template <class S>
__device__ __forceinline__ uint32_t np_hash64(uint64_t c) {
  return static_cast<uint32_t>((c * 0x9e3779b97f4a7c15ull) >> (64 - S::kSlotBits));
}

// exclusive scan of tab[0, kTable) in place by the workgroup (each thread a run of
// kTable / kNpSmallThreads entries); wsum: kNpWaves ints of LDS
template <class S>
__device__ void np_scan(int32_t* tab, int32_t* wsum) {
  constexpr int per = S::kTable / kNpSmallThreads;
  const int t = static_cast<int>(threadIdx.x);
  const int lane = t & (kWave - 1);
  const int wv = t / kWave;
  int v[per];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    v[i] = tab[t * per + i];
    sum += v[i];
  }
  int incl = sum;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  if (lane == kWave - 1) wsum[wv] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wv; ++w) base += wsum[w];
  int run = base + incl - sum;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    tab[t * per + i] = run;
    run += v[i];
  }
  __syncthreads();
}

// one stable pass: elements src[0, n) (round k of thread t at k * 1024 + t) to
// dst by the digit (key >> shift) & (kDigits - 1) of the word's key
template <class S, int DBITS>
__device__ void np_radix_pass(const uint32_t* src, uint32_t* dst, int n, int shift, int32_t* tab,
                              int32_t* wsum) {
  const int t = static_cast<int>(threadIdx.x);
  const int lane = t & (kWave - 1);
  const int wv = t / kWave;
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int i = t; i < S::kTable; i += kNpSmallThreads) tab[i] = 0;
  __syncthreads();
  uint32_t e[S::kPer];
  int dig[S::kPer], rank[S::kPer];
#pragma unroll
  for (int k = 0; k < S::kPer; ++k) {
    const int i = k * kNpSmallThreads + t;
    const bool valid = i < n;
    e[k] = valid ? src[i] : 0u;
    const int d = static_cast<int>((e[k] >> S::kIBits >> shift) & (S::kDigits - 1));
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < DBITS; ++b) {
      const uint64_t bb = __ballot(valid && ((d >> b) & 1));
      m &= ((d >> b) & 1) ? bb : ~bb;
    }
    dig[k] = d;
    rank[k] = __popcll(m & below);
    if (valid && rank[k] == 0) tab[(d * S::kPer + k) * kNpWaves + wv] = __popcll(m);
  }
  __syncthreads();
  np_scan<S>(tab, wsum);
#pragma unroll
  for (int k = 0; k < S::kPer; ++k) {
    const int i = k * kNpSmallThreads + t;
    if (i < n) dst[tab[(dig[k] * S::kPer + k) * kNpWaves + wv] + rank[k]] = e[k];
  }
  __syncthreads();
}

template <int CAP, int DBITS, int PASSES>
__global__ __launch_bounds__(kNpSmallThreads) void np_update_small(int32_t* __restrict__ pool,
                                                                   int64_t* __restrict__ count, int64_t N,
                                                                   int P, const int64_t* __restrict__ src,
                                                                   const int64_t* __restrict__ dst, int n,
                                                                   uint64_t seed, uint64_t call,
                                                                   int32_t* __restrict__ status) {
  using S = NpShape<CAP, DBITS, PASSES>;
  constexpr int kPer = S::kPer;
  constexpr int kIBits = S::kIBits;
  constexpr uint32_t kIMask = (1u << kIBits) - 1;
  extern __shared__ __align__(16) uint8_t lds[];
  int32_t* hsrc = reinterpret_cast<int32_t*>(lds);
  uint32_t* sa = reinterpret_cast<uint32_t*>(lds + S::kLdsSort);
  uint32_t* sb = sa + CAP;
  uint64_t* cells = reinterpret_cast<uint64_t*>(lds);
  int32_t* tab = reinterpret_cast<int32_t*>(lds + S::kLdsTable);
  __shared__ int32_t wsum[kNpWaves];
  const int t = static_cast<int>(threadIdx.x);
  const int lane = t & (kWave - 1);

  // 1. the sources (loaded before any is used) into the source table
  int64_t us[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = k * kNpSmallThreads + t;
    us[k] = i < n ? src[i] : 0;
  }
  for (int i = t; i < S::kSlots; i += kNpSmallThreads) hsrc[i] = kNpEmpty;
  __syncthreads();
  int nbad = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = k * kNpSmallThreads + t;
    const bool bad = i < n && (us[k] < 0 || us[k] >= N);
    nbad += __popcll(__ballot(bad));
    if (i < n) {
      int key = S::kBadKey;
      if (!bad) {
        const int32_t u = static_cast<int32_t>(us[k]);
        uint32_t h = np_hash32<S>(static_cast<uint32_t>(u));
        for (;;) {  // ends: at most CAP of the kSlots slots are ever taken
          int32_t cur = hsrc[h];
          if (cur == kNpEmpty) cur = atomicCAS(&hsrc[h], kNpEmpty, u);
          if (cur == kNpEmpty || cur == u) break;
          h = (h + 1) & (S::kSlots - 1);
        }
        key = static_cast<int>(h);
      }
      sa[i] = static_cast<uint32_t>(key) << kIBits | static_cast<uint32_t>(i);
    }
  }
  if (lane == 0 && nbad != 0 && status != nullptr) atomicAdd(&status[TGX_ST_BAD_EVENT_NODE], nbad);
  __syncthreads();

  // 2. stable sort by key, lowest digit first (the result is back in sa)
  uint32_t* from = sa;
  uint32_t* to = sb;
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    np_radix_pass<S, DBITS>(from, to, n, pass * DBITS, tab, wsum);
    uint32_t* x = from;
    from = to;
    to = x;
  }
  const uint32_t* sorted = from;

  // 3. position p: rank r among the key's edges, the source's count (loaded
  //    before any is used), the decision; the key's last position adds its length
  uint32_t pu[kPer], pj[kPer];
  int pr[kPer], plen[kPer];
  int64_t pc[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int p = k * kNpSmallThreads + t;
    pu[k] = 0;
    pj[k] = 0;
    pr[k] = -1;  // no decision (padding or an out-of-range source)
    plen[k] = 0;
    pc[k] = 0;
    if (p < n) {
      const uint32_t x = sorted[p];
      const uint32_t key = x >> kIBits;
      pj[k] = x & kIMask;
      if (key != static_cast<uint32_t>(S::kBadKey)) {
        const uint32_t first = key << kIBits;
        int lo = 0, hi = p;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (sorted[mid] < first)
            lo = mid + 1;
          else
            hi = mid;
        }
        pu[k] = static_cast<uint32_t>(hsrc[key]);
        pr[k] = p - lo;
        pc[k] = count[pu[k]];
        if (p + 1 == n || (sorted[p + 1] >> kIBits) != key) plen[k] = p - lo + 1;
      }
    }
  }
  uint64_t cell[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    cell[k] = kNpNone;
    if (pr[k] >= 0) {
      const uint32_t j = pj[k];
      const int64_t e = pc[k] + pr[k] + 1;
      int64_t slot = -1;
      if (e <= P) {
        slot = e - 1;
      } else if (uniform01(rand64(seed, call, j, 0)) < static_cast<float>(P) / static_cast<float>(e)) {
        slot = static_cast<int64_t>(rand64(seed, call, j, 1) % static_cast<uint64_t>(P));
      }
      if (slot >= 0) cell[k] = static_cast<uint64_t>(pu[k]) * static_cast<uint64_t>(P) + static_cast<uint64_t>(slot);
    }
  }
  __syncthreads();  // every read of the counts, the sorted words and the source table is done
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (plen[k] > 0) count[pu[k]] += plen[k];

  // 4. the cell table: the largest cell << kIBits | j per cell
  for (int i = t; i < S::kSlots; i += kNpSmallThreads) cells[i] = kNpNone;
  __syncthreads();
  uint32_t ch[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    ch[k] = 0;
    if (cell[k] != kNpNone) {
      const uint64_t word = cell[k] << kIBits | pj[k];
      uint32_t h = np_hash64<S>(cell[k]);
      for (;;) {  // ends: at most CAP of the kSlots slots are ever taken
        const uint64_t old = atomicCAS(reinterpret_cast<unsigned long long*>(&cells[h]),
                                       static_cast<unsigned long long>(kNpNone),
                                       static_cast<unsigned long long>(word));
        if (old == kNpNone) break;
        if ((old >> kIBits) == cell[k]) {
          atomicMax(reinterpret_cast<unsigned long long*>(&cells[h]), static_cast<unsigned long long>(word));
          break;
        }
        h = (h + 1) & (S::kSlots - 1);
      }
      ch[k] = h;
    }
  }
  __syncthreads();
  int64_t val[kPer];
  bool win[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    win[k] = cell[k] != kNpNone && (cells[ch[k]] & kIMask) == pj[k];
    val[k] = win[k] ? dst[pj[k]] : 0;
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (win[k]) pool[cell[k]] = static_cast<int32_t>(val[k]);
}

struct NpLayout {
  RadixScratch r;
  size_t key = 0, idx = 0, ckey = 0, cval = 0, count = 0, sums = 0, total = 0;
};

NpLayout np_layout(int64_t n) {
  NpLayout w;
  w.r = radix_scratch(n);
  const size_t un = static_cast<size_t>(std::max<int64_t>(n, 1));
  w.key = 0;
  w.idx = w.key + 2 * align256(un * 4);
  w.ckey = w.idx + 2 * align256(un * 4);
  w.cval = w.ckey + 2 * align256(un * 8);
  w.count = w.cval + 2 * align256(un * 4);
  w.sums = w.count + w.r.count_bytes;
  w.total = w.sums + w.r.sums_bytes;
  return w;
}

// the caller's cell table of the two-launch update: keys, then latest edges
size_t np_scratch_bytes() { return static_cast<size_t>(kNpCells) * (8 + 4); }

int bits_for(uint64_t max_plus_one) {  // 2^bits - 1 >= max_plus_one - 1 ... and above every valid key
  int bits = 1;
  while (bits < 64 && (uint64_t(1) << bits) < max_plus_one + 1) ++bits;
  return bits;
}

int check_pool(const char* who, const int32_t* pool, const int64_t* count, int64_t N, int32_t P) {
  if (pool == nullptr || count == nullptr) return fail(TGX_ERR_ARG, "%s: pool/count must not be NULL", who);
  if (N <= 0 || N >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "%s: num_nodes %lld outside [1, 2^31)", who, (long long)N);
  if (P < 1 || P > (1 << 20)) return fail(TGX_ERR_LIMIT, "%s: pool_size %d outside [1, 2^20]", who, P);
  return TGX_OK;
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" size_t tgx_negpool_update_workspace_size(int64_t n) {
  if (n < 0) return 0;
  return np_layout(n).total;
}

namespace tgx {
namespace {

int negpool_update(const char* who, int32_t* pool, int64_t* count, int64_t num_nodes, int32_t pool_size,
                   const int64_t* src, const int64_t* dst, int64_t n, uint64_t seed, uint64_t call,
                   const float* u_accept, const int64_t* slot_draw, void* workspace,
                   size_t workspace_bytes, void* scratch, size_t scratch_bytes, int32_t* status,
                   hipStream_t stream) {
  int rc = check_pool(who, pool, count, num_nodes, pool_size);
  if (rc) return rc;
  if (n < 0 || n >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "%s: %lld edges outside [0, 2^31)", who, (long long)n);
  if (n == 0) return TGX_OK;
  if (src == nullptr || dst == nullptr) return fail(TGX_ERR_ARG, "%s: src/dst must not be NULL", who);
  const bool draws = u_accept != nullptr || slot_draw != nullptr;
  if (draws && (u_accept == nullptr || slot_draw == nullptr))
    return fail(TGX_ERR_ARG, "%s: u_accept and slot_draw come together", who);
  const NpLayout w = np_layout(n);
  if (workspace == nullptr || workspace_bytes < w.total)
    return fail(TGX_ERR_ARG, "%s: workspace of %zu bytes needed, got %zu", who, w.total, workspace_bytes);
  if (scratch != nullptr) {
    if (scratch_bytes < np_scratch_bytes())
      return fail(TGX_ERR_ARG, "%s: scratch of %zu bytes needed, got %zu", who, np_scratch_bytes(), scratch_bytes);
    if ((reinterpret_cast<uintptr_t>(scratch) & 255u) != 0)
      return fail(TGX_ERR_ARG, "%s: scratch must be 256-byte aligned", who);
  }
  if (scratch != nullptr && !draws && n <= kNpRankMax) {
    // two launches over the device, the cell table in the caller's scratch
    NpRankParams R{};
    R.src = src;
    R.n = n;
    R.N = num_nodes;
    R.P = static_cast<int>(pool_size);
    R.count = count;
    R.seed = seed;
    R.call = call;
    R.ckey = static_cast<unsigned long long*>(scratch);
    R.cmax = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(scratch) + kNpCells * 8);
    R.rec = static_cast<longlong2*>(workspace);
    R.status = status;
    if (n <= kThreads)
      hipLaunchKernelGGL((np_rank<kThreads, 4>), dim3(1), dim3(kThreads), 0, stream, R);
    else
      hipLaunchKernelGGL((np_rank<kOrderedMaxThreads, 8>), dim3(static_cast<unsigned>(cdiv(n, kOrderedMaxThreads))),
                         dim3(kOrderedMaxThreads), 0, stream, R);
    if ((rc = check_launch("np_rank"))) return rc;
    hipLaunchKernelGGL(np_commit, dim3(static_cast<unsigned>(cdiv(n, kThreads))), dim3(kThreads), 0, stream,
                       static_cast<const longlong2*>(R.rec), src, dst, n, R.ckey, R.cmax, pool, count);
    return check_launch("np_commit");
  }
  if (n <= 8192 && !draws) {
    // one workgroup: the 4,096-edge shape, or the 8,192-edge one (three digit passes)
    static std::once_flag attr_once;
    std::call_once(attr_once, [] {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(np_update_small<4096, 7, 2>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(NpSmall::kLds));
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(np_update_small<8192, 5, 3>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(NpMid::kLds));
      (void)hipGetLastError();
    });
    if (n <= 4096)
      hipLaunchKernelGGL((np_update_small<4096, 7, 2>), dim3(1), dim3(kNpSmallThreads), NpSmall::kLds, stream,
                         pool, count, num_nodes, static_cast<int>(pool_size), src, dst, static_cast<int>(n), seed,
                         call, status);
    else
      hipLaunchKernelGGL((np_update_small<8192, 5, 3>), dim3(1), dim3(kNpSmallThreads), NpMid::kLds, stream,
                         pool, count, num_nodes, static_cast<int>(pool_size), src, dst, static_cast<int>(n), seed,
                         call, status);
    return check_launch("np_update_small");
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const size_t un = static_cast<size_t>(n);
  uint32_t* key[2] = {reinterpret_cast<uint32_t*>(ws + w.key), reinterpret_cast<uint32_t*>(ws + w.key + align256(un * 4))};
  uint32_t* idx[2] = {reinterpret_cast<uint32_t*>(ws + w.idx), reinterpret_cast<uint32_t*>(ws + w.idx + align256(un * 4))};
  uint64_t* ck[2] = {reinterpret_cast<uint64_t*>(ws + w.ckey), reinterpret_cast<uint64_t*>(ws + w.ckey + align256(un * 8))};
  uint32_t* cv[2] = {reinterpret_cast<uint32_t*>(ws + w.cval), reinterpret_cast<uint32_t*>(ws + w.cval + align256(un * 4))};
  uint32_t* cnt = reinterpret_cast<uint32_t*>(ws + w.count);
  uint32_t* sums = reinterpret_cast<uint32_t*>(ws + w.sums);
  const dim3 g1(static_cast<unsigned>(cdiv(n, kThreads)));
  hipLaunchKernelGGL(np_keys, g1, dim3(kThreads), 0, stream, src, n, num_nodes, key[0], idx[0], status);
  if ((rc = check_launch("np_keys"))) return rc;
  int cur = 0;
  if ((rc = radix_sort<uint32_t>(key, idx, cur, n, bits_for(static_cast<uint64_t>(num_nodes)), w.r, cnt,
                                 sums, stream)))
    return rc;
  hipLaunchKernelGGL(np_decide, g1, dim3(kThreads), 0, stream, static_cast<const uint32_t*>(key[cur]),
                     static_cast<const uint32_t*>(idx[cur]), n, static_cast<const int64_t*>(count),
                     static_cast<int>(pool_size), seed, call, u_accept, slot_draw, ck[0], cv[0]);
  if ((rc = check_launch("np_decide"))) return rc;
  int ccur = 0;
  const uint64_t cells = static_cast<uint64_t>(num_nodes) * static_cast<uint64_t>(pool_size);
  if ((rc = radix_sort<uint64_t>(ck, cv, ccur, n, bits_for(cells), w.r, cnt, sums, stream))) return rc;
  hipLaunchKernelGGL(np_write, g1, dim3(kThreads), 0, stream, static_cast<const uint64_t*>(ck[ccur]),
                     static_cast<const uint32_t*>(cv[ccur]), n, dst, pool);
  if ((rc = check_launch("np_write"))) return rc;
  hipLaunchKernelGGL(np_count, g1, dim3(kThreads), 0, stream, static_cast<const uint32_t*>(key[cur]), n,
                     count);
  return check_launch("np_count");
}

int negpool_sample(const char* who, const int32_t* pool, const int64_t* count, int64_t num_nodes,
                   int32_t pool_size, const int64_t* src, int64_t n, uint64_t seed, uint64_t call,
                   const float* u_slot, int64_t* out, int32_t* status, hipStream_t stream) {
  int rc = check_pool(who, pool, count, num_nodes, pool_size);
  if (rc) return rc;
  if (n < 0) return fail(TGX_ERR_ARG, "%s: negative size", who);
  if (n == 0) return TGX_OK;
  if (src == nullptr || out == nullptr) return fail(TGX_ERR_ARG, "%s: src/out must not be NULL", who);
  hipLaunchKernelGGL(np_sample, dim3(static_cast<unsigned>(cdiv(n, kThreads))), dim3(kThreads), 0, stream,
                     pool, count, num_nodes, static_cast<int>(pool_size), src, n, seed, call, u_slot, out,
                     status);
  return check_launch("np_sample");
}

}  // namespace
}  // namespace tgx

extern "C" int tgx_negpool_update(int32_t* pool, int64_t* count, int64_t num_nodes, int32_t pool_size,
                                  const int64_t* src, const int64_t* dst, int64_t n, uint64_t seed,
                                  uint64_t call, void* workspace, size_t workspace_bytes, void* scratch,
                                  size_t scratch_bytes, int32_t* status, void* stream) {
  return negpool_update("tgx_negpool_update", pool, count, num_nodes, pool_size, src, dst, n, seed, call,
                        nullptr, nullptr, workspace, workspace_bytes, scratch, scratch_bytes, status,
                        static_cast<hipStream_t>(stream));
}

extern "C" size_t tgx_negpool_scratch_size(void) { return np_scratch_bytes(); }

extern "C" int tgx_negpool_update_draws(int32_t* pool, int64_t* count, int64_t num_nodes, int32_t pool_size,
                                        const int64_t* src, const int64_t* dst, int64_t n,
                                        const float* u_accept, const int64_t* slot_draw, void* workspace,
                                        size_t workspace_bytes, int32_t* status, void* stream) {
  if (n > 0 && (u_accept == nullptr || slot_draw == nullptr))
    return fail(TGX_ERR_ARG, "tgx_negpool_update_draws: u_accept/slot_draw must not be NULL");
  return negpool_update("tgx_negpool_update_draws", pool, count, num_nodes, pool_size, src, dst, n, 0, 0,
                        u_accept, slot_draw, workspace, workspace_bytes, nullptr, 0, status,
                        static_cast<hipStream_t>(stream));
}

extern "C" int tgx_negpool_sample(const int32_t* pool, const int64_t* count, int64_t num_nodes,
                                  int32_t pool_size, const int64_t* src, int64_t n, uint64_t seed,
                                  uint64_t call, int64_t* out, int32_t* status, void* stream) {
  return negpool_sample("tgx_negpool_sample", pool, count, num_nodes, pool_size, src, n, seed, call, nullptr,
                        out, status, static_cast<hipStream_t>(stream));
}

extern "C" int tgx_negpool_sample_draws(const int32_t* pool, const int64_t* count, int64_t num_nodes,
                                        int32_t pool_size, const int64_t* src, int64_t n, const float* u_slot,
                                        int64_t* out, int32_t* status, void* stream) {
  if (n > 0 && u_slot == nullptr) return fail(TGX_ERR_ARG, "tgx_negpool_sample_draws: u_slot must not be NULL");
  return negpool_sample("tgx_negpool_sample_draws", pool, count, num_nodes, pool_size, src, n, 0, 0, u_slot,
                        out, status, static_cast<hipStream_t>(stream));
}
