// Kernel (a): ring-buffer update for one batch of events.
//
// Semantics (reference tgengine/core/temporal_graph.py:123-129 and
// _append_overflow :351-387): the batch of b undirected events becomes n = 2b
// directed entries in concatenation order i = [src->dst for every event,
// dst->src for every event].  Grouped by `from` node in that order, each node
// with c entries keeps its last min(c, B); the m-th kept entry goes to slot
// (write_pos + m) % B and write_pos grows by min(c, B).
//
// Design.  Two launches on the caller's stream:
//   1. ring_plan: ONE workgroup of 512 threads.  A stable LSD radix sort with
//      4-bit digits orders the entry indices by node id (stable, so concat
//      order survives inside a node); two block scans find every run's start
//      and end; each entry gets its destination slot u*B + s (or -1 when it is
//      not among the last B of its node), and every run head advances
//      write_pos.  For n <= 16384 the keys (64 KB) and the two index buffers
//      (2 x 32 KB, uint16) live in LDS; larger batches use the same code on a
//      global-memory workspace.
//   2. ring_write: wide copy of ids / times / edge ids / feature rows into
//      the planned slots, 16-byte vector accesses when the row allows it.
// The sort is integer work on one CU by design: a batch holds at most a few
// thousand distinct nodes, while a device-wide sort would cost several
// launches; the feature bytes move in the wide kernel.
#include "tgx_internal.h"

namespace tgx {
namespace {

constexpr int kPlanThreads = 512;
constexpr int kPlanWaves = kPlanThreads / kWave;
constexpr int kLdsMaxEntries = 16384;

__device__ __forceinline__ int pad32(int p) { return p + (p >> 5); }

// (write_pos + off) % B for write_pos >= 0, 0 <= off < B; 32-bit arithmetic
// whenever the value fits (B is usually a power of two)
__device__ __forceinline__ int64_t ring_slot(int64_t w, int off, int B) {
  const uint64_t x = static_cast<uint64_t>(w) + static_cast<uint64_t>(off);
  if ((B & (B - 1)) == 0) return static_cast<int64_t>(x & static_cast<uint64_t>(B - 1));
  if (x < (uint64_t(1) << 32)) return static_cast<int64_t>(static_cast<uint32_t>(x) % static_cast<uint32_t>(B));
  return static_cast<int64_t>(x % static_cast<uint64_t>(B));
}


// ---------------------------------------------------------------------------
// digit counters, one column per thread.
//   packed: word (d>>1)*T + t holds the 16-bit counters of digits 2j, 2j+1
//   wide:   word d*T + t holds the 32-bit counter of digit d
// ---------------------------------------------------------------------------
template <bool kPacked>
struct Counters {
  static constexpr int kWords = kPacked ? 8 : 16;
  uint32_t* w;
  __device__ __forceinline__ void zero_own(int t) {
#pragma unroll
    for (int j = 0; j < kWords; ++j) w[j * kPlanThreads + t] = 0u;
  }
  __device__ __forceinline__ void add1(uint32_t d, int t) {
    if (kPacked)
      atomicAdd(&w[(d >> 1) * kPlanThreads + t], 1u << ((d & 1u) * 16u));
    else
      atomicAdd(&w[d * kPlanThreads + t], 1u);
  }
  __device__ __forceinline__ uint32_t fetch_add1(uint32_t d, int t) {
    if (kPacked) {
      const uint32_t sh = (d & 1u) * 16u;
      const uint32_t old = atomicAdd(&w[(d >> 1) * kPlanThreads + t], 1u << sh);
      return (old >> sh) & 0xFFFFu;
    } else {
      return atomicAdd(&w[d * kPlanThreads + t], 1u);
    }
  }
};

__device__ __forceinline__ uint32_t wave_incl_scan_add(uint32_t x, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  return x;
}

// Block-wide exclusive scan of the per-(digit, thread) counters in digit-major
// order; the counters are replaced by the scatter offsets.
template <bool kPacked>
__device__ __forceinline__ void scan_counters(Counters<kPacked> cnt, uint32_t* wsum, int t) {
  constexpr int W = Counters<kPacked>::kWords;
  const int lane = t & (kWave - 1), wv = t / kWave;
  uint32_t c[W], x[W];
#pragma unroll
  for (int j = 0; j < W; ++j) {
    c[j] = cnt.w[j * kPlanThreads + t];
    x[j] = wave_incl_scan_add(c[j], lane);
  }
  if (lane == kWave - 1) {
#pragma unroll
    for (int j = 0; j < W; ++j) wsum[wv * W + j] = x[j];
  }
  __syncthreads();
  uint32_t tot[W];
#pragma unroll
  for (int j = 0; j < W; ++j) tot[j] = 0u;
  for (int w2 = 0; w2 < kPlanWaves; ++w2) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const uint32_t s = wsum[w2 * W + j];
      if (w2 < wv) x[j] += s;
      tot[j] += s;
    }
  }
  // digit totals -> exclusive digit bases
  uint32_t base[16];
  uint32_t run = 0;
#pragma unroll
  for (int d = 0; d < 16; ++d) {
    base[d] = run;
    const uint32_t td = kPacked ? ((tot[d >> 1] >> ((d & 1) * 16)) & 0xFFFFu) : tot[d];
    run += td;
  }
#pragma unroll
  for (int j = 0; j < W; ++j) {
    const uint32_t ex = x[j] - c[j];  // fieldwise exclusive (no borrow: x >= c per field)
    if (kPacked) {
      const uint32_t lo = base[2 * j] + (ex & 0xFFFFu);
      const uint32_t hi = base[2 * j + 1] + (ex >> 16);
      cnt.w[j * kPlanThreads + t] = lo | (hi << 16);
    } else {
      cnt.w[j * kPlanThreads + t] = base[j] + ex;
    }
  }
}

// exclusive max-scan (forward) of one int per thread
__device__ __forceinline__ int block_excl_max(int v, int* sh, int t) {
  const int lane = t & (kWave - 1), wv = t / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x = max(x, y);
  }
  if (lane == kWave - 1) sh[wv] = x;
  __syncthreads();
  int carry = -1;
  for (int w2 = 0; w2 < wv; ++w2) carry = max(carry, sh[w2]);
  int ex = __shfl_up(x, 1, kWave);
  if (lane == 0) ex = -1;
  __syncthreads();
  return max(carry, ex);
}

// exclusive min-scan from the right (carry = min over threads > t)
__device__ __forceinline__ int block_excl_min_rev(int v, int* sh, int t, int identity) {
  const int lane = t & (kWave - 1), wv = t / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_down(x, off, kWave);
    if (lane + off < kWave) x = min(x, y);
  }
  if (lane == 0) sh[wv] = x;
  __syncthreads();
  int carry = identity;
  for (int w2 = wv + 1; w2 < kPlanWaves; ++w2) carry = min(carry, sh[w2]);
  int ex = __shfl_down(x, 1, kWave);
  if (lane == kWave - 1) ex = identity;
  __syncthreads();
  return min(carry, ex);
}

template <typename IdxT, bool kPacked>
__device__ __forceinline__ void plan_body(const int64_t* __restrict__ src,
                                          const int64_t* __restrict__ dst,
                                          const double* __restrict__ time, int n, int b,
                                          int64_t N, int B, int64_t* __restrict__ wp,
                                          int64_t* __restrict__ dest, uint32_t* keys, IdxT* pa,
                                          IdxT* pb, uint32_t* cnt_words, uint32_t* wsum,
                                          int* ish, double* dsh, int32_t* status) {
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1), wv = t / kWave;
  Counters<kPacked> cnt{cnt_words};

  // ---- keys (node id, N = invalid sentinel) and diagnostics ----
  int bad = 0;
  for (int i = t; i < n; i += kPlanThreads) {
    const int64_t u = i < b ? src[i] : dst[i - b];
    uint32_t k;
    if (u < 0 || u >= N) {
      k = static_cast<uint32_t>(N);
      ++bad;
    } else {
      k = static_cast<uint32_t>(u);
    }
    keys[i] = k;
    pa[i] = static_cast<IdxT>(i);
  }
  double mx = -__builtin_inf();
  for (int i = t; i < b; i += kPlanThreads) mx = fmax(mx, time[i]);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    bad += __shfl_xor(bad, off, kWave);
    mx = fmax(mx, __shfl_xor(mx, off, kWave));
  }
  if (lane == 0) {
    ish[wv] = bad;
    dsh[wv] = mx;
  }
  __syncthreads();
  if (t == 0 && status != nullptr) {
    int tb = 0;
    double tm = -__builtin_inf();
    for (int w2 = 0; w2 < kPlanWaves; ++w2) {
      tb += ish[w2];
      tm = fmax(tm, dsh[w2]);
    }
    if (tb) atomicAdd(&status[TGX_ST_BAD_EVENT_NODE], tb);
    // reference key from*(int(max t)+2)+i is lexicographic iff int(max t)+2 > n-1
    if (!(trunc(tm) > static_cast<double>(n - 3))) atomicAdd(&status[TGX_ST_KEY_COLLISION], 1);
  }
  __syncthreads();

  // ---- stable LSD radix sort of entry indices by key, 4-bit digits ----
  const int nbits = 32 - __clz(static_cast<uint32_t>(N));  // covers the sentinel N
  const int passes = (nbits + 3) / 4;
  const int E = (n + kPlanThreads - 1) / kPlanThreads;
  const int beg = min(n, t * E);
  const int end = min(n, beg + E);
  IdxT* in = pa;
  IdxT* out = pb;
  for (int ps = 0; ps < passes; ++ps) {
    const int shift = ps * 4;
    cnt.zero_own(t);
    for (int p = beg; p < end; ++p) cnt.add1((keys[in[p]] >> shift) & 15u, t);
    __syncthreads();
    scan_counters<kPacked>(cnt, wsum, t);
    __syncthreads();
    for (int p = beg; p < end; ++p) {
      const IdxT v = in[p];
      const uint32_t pos = cnt.fetch_add1((keys[v] >> shift) & 15u, t);
      out[pos] = v;
    }
    __syncthreads();
    IdxT* tmp = in;
    in = out;
    out = tmp;
  }
  // `in` = sorted permutation, `out` = free buffer

  // ---- run starts (forward) ----
  int last_head = -1, first_head = n;
  for (int p = beg; p < end; ++p) {
    const bool head = (p == 0) || (keys[in[p]] != keys[in[p - 1]]);
    if (head) {
      last_head = p;
      if (first_head == n) first_head = p;
    }
  }
  int start = block_excl_max(last_head, ish, t);
  const int next_head_after = block_excl_min_rev(first_head, ish, t, n);
  for (int p = beg; p < end; ++p) {
    const bool head = (p == 0) || (keys[in[p]] != keys[in[p - 1]]);
    if (head) start = p;
    out[p] = static_cast<IdxT>(start);
  }
  // ---- run ends (backward) and destinations ----
  int run_end = next_head_after;
  for (int p = end - 1; p >= beg; --p) {
    const int s = static_cast<int>(out[p]);
    const uint32_t u = keys[in[p]];
    const int idx = static_cast<int>(in[p]);
    const int c = run_end - s;
    const int kept = min(c, B);
    const int m = p - s;
    int64_t dslot = -1;
    if (u < static_cast<uint32_t>(N) && m >= c - kept) {
      const int64_t w0 = wp[u];
      const int64_t slot = ring_slot(w0, m - (c - kept), B);
      dslot = static_cast<int64_t>(u) * B + slot;
    }
    dest[idx] = dslot;
    if (p == s) {
      out[p] = static_cast<IdxT>(kept);  // run head keeps the kept count
      run_end = s;
    }
  }
  __syncthreads();
  // ---- advance write_pos once per node ----
  for (int p = beg; p < end; ++p) {
    const uint32_t u = keys[in[p]];
    const bool head = (p == 0) || (u != keys[in[p - 1]]);
    if (head && u < static_cast<uint32_t>(N)) wp[u] += static_cast<int64_t>(out[p]);
  }
}

// ---------------------------------------------------------------------------
// Fast plan for n <= 16384 entries: one workgroup of 1024 threads, each
// owning 16 consecutive positions of the array in registers ("blocked"
// arrangement).  Per 4-bit pass: digits and in-thread ranks in registers
// (8-bit counters packed in two u64), one block-wide scan of the 16 digit
// counts (16-bit fields packed in four u64), a scatter of (key, index) into
// LDS and a gather back into registers.  Only the exchange arrays and the
// per-thread digit offsets live in LDS (64 + 32 + 32 KB).
// ---------------------------------------------------------------------------
constexpr int kFT = 512;              // threads
constexpr int kFW = kFT / kWave;      // waves
constexpr int kFE = 32;               // items per thread

__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t x, int off) {
  const uint32_t lo = __shfl_up(static_cast<uint32_t>(x), off, kWave);
  const uint32_t hi = __shfl_up(static_cast<uint32_t>(x >> 32), off, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <int NW>
__device__ __forceinline__ int block_excl_max_n(int v, int* sh, int t) {
  const int lane = t & (kWave - 1), wv = t / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x = max(x, y);
  }
  if (lane == kWave - 1) sh[wv] = x;
  __syncthreads();
  int carry = -1;
  for (int w2 = 0; w2 < wv; ++w2) carry = max(carry, sh[w2]);
  int ex = __shfl_up(x, 1, kWave);
  if (lane == 0) ex = -1;
  __syncthreads();
  return max(carry, ex);
}

template <int NW>
__device__ __forceinline__ int block_excl_min_rev_n(int v, int* sh, int t, int identity) {
  const int lane = t & (kWave - 1), wv = t / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_down(x, off, kWave);
    if (lane + off < kWave) x = min(x, y);
  }
  if (lane == 0) sh[wv] = x;
  __syncthreads();
  int carry = identity;
  for (int w2 = wv + 1; w2 < NW; ++w2) carry = min(carry, sh[w2]);
  int ex = __shfl_down(x, 1, kWave);
  if (lane == kWave - 1) ex = identity;
  __syncthreads();
  return min(carry, ex);
}

__global__ __launch_bounds__(kFT) void ring_plan_fast(
    const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
    const double* __restrict__ time, int n, int b, int64_t N, int B, int64_t* __restrict__ wp,
    int64_t* __restrict__ dest, int32_t* status) {
  // exchange arrays, padded by one entry per 32 (index p + p/32) so the
  // blocked reads t*E + e spread over the LDS banks
  __shared__ uint32_t xk[kFT * kFE + kFT * kFE / 32];
  __shared__ uint16_t xv[kFT * kFE + kFT * kFE / 32];
  __shared__ uint16_t offs[16 * kFT];
  __shared__ uint64_t wsum[kFW * 4];
  __shared__ int ish[kFW];
  __shared__ double dsh[kFW];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1), wv = t / kWave;
  const int E = (n + kFT - 1) / kFT;
  const uint32_t kInvalid = static_cast<uint32_t>(N);
  const uint32_t kPad = static_cast<uint32_t>(N) + 1u;

  uint32_t k[kFE], v[kFE];
  int bad = 0;
#pragma unroll
  for (int e = 0; e < kFE; ++e) {
    const int p = t * E + e;
    k[e] = kPad;
    v[e] = static_cast<uint32_t>(p);
    if (e < E && p < n) {
      const int64_t u = p < b ? src[p] : dst[p - b];
      if (u < 0 || u >= N) {
        k[e] = kInvalid;
        ++bad;
      } else {
        k[e] = static_cast<uint32_t>(u);
      }
    }
  }
  double mx = -__builtin_inf();
  for (int i = t; i < b; i += kFT) mx = fmax(mx, time[i]);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    bad += __shfl_xor(bad, off, kWave);
    mx = fmax(mx, __shfl_xor(mx, off, kWave));
  }
  if (lane == 0) {
    ish[wv] = bad;
    dsh[wv] = mx;
  }
  __syncthreads();
  if (t == 0 && status != nullptr) {
    int tb = 0;
    double tm = -__builtin_inf();
    for (int w2 = 0; w2 < kFW; ++w2) {
      tb += ish[w2];
      tm = fmax(tm, dsh[w2]);
    }
    if (tb) atomicAdd(&status[TGX_ST_BAD_EVENT_NODE], tb);
    if (!(trunc(tm) > static_cast<double>(n - 3))) atomicAdd(&status[TGX_ST_KEY_COLLISION], 1);
  }
  __syncthreads();

  const int nbits = 32 - __clz(kPad);
  for (int shift = 0; shift < nbits; shift += 4) {
    // per-thread digit counts (8-bit fields: digits 0-7 in c0, 8-15 in c1)
    uint64_t c0 = 0, c1 = 0;
#pragma unroll
    for (int e = 0; e < kFE; ++e) {
      if (e < E) {
        const uint32_t d = (k[e] >> shift) & 15u;
        const uint64_t inc = uint64_t(1) << ((d & 7u) * 8u);
        if (d < 8u) c0 += inc; else c1 += inc;
      }
    }
    // counts as four u64 of 16-bit fields (digits 4j..4j+3)
    uint64_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t c = j < 2 ? c0 : c1;
      const int b0 = (j & 1) * 32;
      q[j] = ((c >> b0) & 0xFFu) | (((c >> (b0 + 8)) & 0xFFu) << 16) |
             (((c >> (b0 + 16)) & 0xFFu) << 32) | (((c >> (b0 + 24)) & 0xFFu) << 48);
    }
    uint64_t x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = q[j];
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const uint64_t y = shfl_up_u64(x[j], off);
        if (lane >= off) x[j] += y;
      }
    }
    if (lane == kWave - 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) wsum[wv * 4 + j] = x[j];
    }
    __syncthreads();
    uint64_t tot[4] = {0, 0, 0, 0};
    for (int w2 = 0; w2 < kFW; ++w2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t s2 = wsum[w2 * 4 + j];
        if (w2 < wv) x[j] += s2;
        tot[j] += s2;
      }
    }
    uint32_t run = 0;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      const uint32_t ex = static_cast<uint32_t>(((x[d >> 2] - q[d >> 2]) >> ((d & 3) * 16)) & 0xFFFFu);
      offs[d * kFT + t] = static_cast<uint16_t>(run + ex);
      run += static_cast<uint32_t>((tot[d >> 2] >> ((d & 3) * 16)) & 0xFFFFu);
    }
    // scatter; in-thread ranks are recounted in the same order
    c0 = 0;
    c1 = 0;
#pragma unroll
    for (int e = 0; e < kFE; ++e) {
      if (e < E) {
        const uint32_t d = (k[e] >> shift) & 15u;
        const uint32_t sh = (d & 7u) * 8u;
        const uint64_t c = d < 8u ? c0 : c1;
        const uint32_t rk = static_cast<uint32_t>((c >> sh) & 0xFFu);
        const uint64_t cn = c + (uint64_t(1) << sh);
        if (d < 8u) c0 = cn; else c1 = cn;
        const uint32_t pos = static_cast<uint32_t>(offs[d * kFT + t]) + rk;
        xk[pad32(pos)] = k[e];
        xv[pad32(pos)] = static_cast<uint16_t>(v[e]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kFE; ++e) {
      if (e < E) {
        k[e] = xk[pad32(t * E + e)];
        v[e] = xv[pad32(t * E + e)];
      }
    }
    __syncthreads();
  }

  // ---- runs of equal keys over the sorted positions ----
  const int L = kFT * E;
  int last_head = -1, first_head = L;
  uint32_t prevk = (t == 0) ? 0xFFFFFFFFu : xk[pad32(t * E - 1)];
  uint32_t heads = 0;  // bit e: position t*E+e starts a run
#pragma unroll
  for (int e = 0; e < kFE; ++e) {
    if (e < E) {
      const int p = t * E + e;
      if (p == 0 || k[e] != prevk) {
        heads |= 1u << e;
        last_head = p;
        if (first_head == L) first_head = p;
      }
      prevk = k[e];
    }
  }
  int start = block_excl_max_n<kFW>(last_head, ish, t);
  const int next_after = block_excl_min_rev_n<kFW>(first_head, ish, t, L);
  int st[kFE];
#pragma unroll
  for (int e = 0; e < kFE; ++e) {
    if (e < E && ((heads >> e) & 1u)) start = t * E + e;
    st[e] = start;
  }
  int run_end = next_after;
#pragma unroll
  for (int e = kFE - 1; e >= 0; --e) {
    if (e < E) {
      const int p = t * E + e;
      const int c = run_end - st[e];
      const int kept = min(c, B);
      const int m = p - st[e];
      if (static_cast<int>(v[e]) < n) {
        int64_t dslot = -1;
        if (k[e] < kInvalid && m >= c - kept) {
          const int64_t slot = ring_slot(wp[k[e]], m - (c - kept), B);
          dslot = static_cast<int64_t>(k[e]) * B + slot;
        }
        dest[v[e]] = dslot;
      }
      if ((heads >> e) & 1u) {
        xv[pad32(p)] = static_cast<uint16_t>(kept);  // the sorted indices now live in registers
        run_end = p;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kFE; ++e) {
    if (e < E && ((heads >> e) & 1u) && k[e] < kInvalid) wp[k[e]] += xv[pad32(t * E + e)];
  }
}

__global__ __launch_bounds__(kPlanThreads) void ring_plan_global(
    const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
    const double* __restrict__ time, int n, int b, int64_t N, int B, int64_t* __restrict__ wp,
    int64_t* __restrict__ dest, uint32_t* gkeys, uint32_t* gpa, uint32_t* gpb,
    int32_t* status) {
  __shared__ uint32_t cnt[16 * kPlanThreads];
  __shared__ uint32_t wsum[kPlanWaves * 16];
  __shared__ int ish[kPlanWaves];
  __shared__ double dsh[kPlanWaves];
  plan_body<uint32_t, false>(src, dst, time, n, b, N, B, wp, dest, gkeys, gpa, gpb, cnt, wsum,
                             ish, dsh, status);
}

template <int VEC>
struct VecT;
template <>
struct VecT<16> {
  using T = uint4;
};
template <>
struct VecT<4> {
  using T = uint32_t;
};
template <>
struct VecT<2> {
  using T = uint16_t;
};

template <int VEC>
__global__ __launch_bounds__(256) void ring_write(
    const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
    const double* __restrict__ time, const uint8_t* __restrict__ feat, int64_t b,
    int64_t eid_base, int64_t row_bytes, const int64_t* __restrict__ dest,
    int32_t* __restrict__ ids, double* __restrict__ times, uint8_t* __restrict__ feats,
    int64_t* __restrict__ eids, int tpe_log2) {
  using V = typename VecT<VEC>::T;
  const int tpe = 1 << tpe_log2;
  const int epb = 256 >> tpe_log2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * epb + (threadIdx.x >> tpe_log2);
  const int l = threadIdx.x & (tpe - 1);
  if (i >= 2 * b) return;
  const int64_t slot = dest[i];
  if (slot < 0) return;
  const int64_t e = i < b ? i : i - b;
  if (l == 0) {
    ids[slot] = static_cast<int32_t>(i < b ? dst[e] : src[e]);
    times[slot] = time[e];
    if (eids != nullptr) eids[slot] = eid_base + e;
  }
  const int64_t nv = row_bytes / VEC;
  V* drow = reinterpret_cast<V*>(feats + slot * row_bytes);
  if (feat != nullptr) {
    const V* srow = reinterpret_cast<const V*>(feat + e * row_bytes);
    for (int64_t c = l; c < nv; c += tpe) drow[c] = srow[c];
  } else {
    for (int64_t c = l; c < nv; c += tpe) drow[c] = V{};
  }
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" size_t tgx_ring_append_workspace_size(int64_t b) {
  if (b <= 0) return 256;
  const int64_t n = 2 * b;
  size_t bytes = align256(static_cast<size_t>(n) * sizeof(int64_t));
  if (n > kLdsMaxEntries) bytes += 3 * align256(static_cast<size_t>(n) * sizeof(uint32_t));
  return bytes;
}

extern "C" int tgx_ring_append(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                               const double* time, const void* feat, int64_t b,
                               int64_t eid_base, void* workspace, size_t workspace_bytes,
                               int32_t* status, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (ring == nullptr) return fail(TGX_ERR_ARG, "tgx_ring_append: ring is NULL");
  if (b < 0) return fail(TGX_ERR_ARG, "tgx_ring_append: negative batch size %lld", (long long)b);
  if (b == 0) return TGX_OK;
  if (src == nullptr || dst == nullptr || time == nullptr)
    return fail(TGX_ERR_ARG, "tgx_ring_append: src/dst/time must not be NULL");
  if (ring->ids == nullptr || ring->times == nullptr || ring->write_pos == nullptr ||
      (ring->feats == nullptr && ring->feat_dim > 0))
    return fail(TGX_ERR_ARG, "tgx_ring_append: ring arrays must not be NULL");
  const int esz = feat_elem_bytes(ring->feat_dtype);
  if (esz == 0) return fail(TGX_ERR_DTYPE, "tgx_ring_append: unsupported feat dtype %d", ring->feat_dtype);
  if (ring->num_nodes <= 0 || ring->num_nodes >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "tgx_ring_append: num_nodes %lld outside [1, 2^31)",
                (long long)ring->num_nodes);
  if (ring->slots <= 0 || ring->slots > (1 << 15))
    return fail(TGX_ERR_LIMIT, "tgx_ring_append: slots %d outside [1, 32768]", ring->slots);
  if (ring->feat_dim < 0) return fail(TGX_ERR_ARG, "tgx_ring_append: negative feat_dim");
  const int64_t n = 2 * b;
  if (n >= (int64_t(1) << 30)) return fail(TGX_ERR_LIMIT, "tgx_ring_append: batch too large");
  const size_t need = tgx_ring_append_workspace_size(b);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(TGX_ERR_ARG, "tgx_ring_append: workspace of %zu bytes needed, got %zu", need,
                workspace_bytes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int64_t* dest = reinterpret_cast<int64_t*>(ws);

  if (n <= kLdsMaxEntries) {
    hipLaunchKernelGGL(ring_plan_fast, dim3(1), dim3(kFT), 0, stream, src, dst, time,
                       static_cast<int>(n), static_cast<int>(b), ring->num_nodes, ring->slots,
                       ring->write_pos, dest, status);
  } else {
    uint8_t* p = ws + align256(static_cast<size_t>(n) * sizeof(int64_t));
    uint32_t* gkeys = reinterpret_cast<uint32_t*>(p);
    p += align256(static_cast<size_t>(n) * 4);
    uint32_t* gpa = reinterpret_cast<uint32_t*>(p);
    p += align256(static_cast<size_t>(n) * 4);
    uint32_t* gpb = reinterpret_cast<uint32_t*>(p);
    hipLaunchKernelGGL(ring_plan_global, dim3(1), dim3(kPlanThreads), 0, stream, src, dst, time,
                       static_cast<int>(n), static_cast<int>(b), ring->num_nodes, ring->slots,
                       ring->write_pos, dest, gkeys, gpa, gpb, status);
  }
  int rc = check_launch("ring_plan");
  if (rc) return rc;

  const int64_t row_bytes = static_cast<int64_t>(ring->feat_dim) * esz;
  int vec = 2;
  if (row_bytes % 16 == 0 && aligned16(ring->feats) && (feat == nullptr || aligned16(feat)))
    vec = 16;
  else if (row_bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(ring->feats) & 3u) == 0 &&
           (feat == nullptr || (reinterpret_cast<uintptr_t>(feat) & 3u) == 0))
    vec = 4;
  const int64_t nchunks = row_bytes / vec;
  int tpe_log2 = 0;
  while ((int64_t(1) << tpe_log2) < nchunks && tpe_log2 < 6) ++tpe_log2;
  const int epb = 256 >> tpe_log2;
  const int64_t grid = (n + epb - 1) / epb;
  const uint8_t* fb = static_cast<const uint8_t*>(feat);
  uint8_t* rf = static_cast<uint8_t*>(ring->feats);
  switch (vec) {
    case 16:
      hipLaunchKernelGGL(ring_write<16>, dim3(grid), dim3(256), 0, stream, src, dst, time, fb, b,
                         eid_base, row_bytes, dest, ring->ids, ring->times, rf, ring->eids, tpe_log2);
      break;
    case 4:
      hipLaunchKernelGGL(ring_write<4>, dim3(grid), dim3(256), 0, stream, src, dst, time, fb, b,
                         eid_base, row_bytes, dest, ring->ids, ring->times, rf, ring->eids, tpe_log2);
      break;
    default:
      hipLaunchKernelGGL(ring_write<2>, dim3(grid), dim3(256), 0, stream, src, dst, time, fb, b,
                         eid_base, row_bytes, dest, ring->ids, ring->times, rf, ring->eids, tpe_log2);
      break;
  }
  return check_launch("ring_write");
}
