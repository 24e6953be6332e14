// Frozen-CSR build (reference TemporalGraph.freeze_csr, temporal_graph.py:133-181).
//
// The n directed entries of the pre-freeze advance() calls, in build order j
// (per call: [src->dst for every event, dst->src for every event]), are sorted
// stably by time and then stably by node, so a node's entries end up
// time-ascending with ties in build order (the reference's two stable
// argsorts, :156-158).  The same permutation comes out of a stable LSD radix
// sort: eight 8-bit passes over an order-preserving 64-bit image of the time,
// then ceil(log2 N / 8) passes over the node id.
//
// The passes are tgx_radix.h's.  Then offsets[u] = lower_bound(sorted nodes, u), and one gather writes the
// ids, times, edge ids and feature rows (16-byte vectors where aligned).
//
// Event pairs (TGX_CSR_EVENT_PAIRS): the caller hands the events themselves in
// an order whose entries 2k, 2k+1 are already the stable time order of the
// build order (a time-ordered stream); the time passes are skipped and the
// kernels read an entry's node, neighbour, time and event from its event.
#include "tgx_radix.h"

namespace tgx {
namespace {

// order-preserving image of a float64: -0.0 maps to +0.0 and every NaN to one
// NaN above +inf, so ties are exactly the ties of a float comparison
__device__ __forceinline__ uint64_t time_key(double t) {
  uint64_t u;
  if (t != t)
    u = 0x7ff8000000000000ull;
  else if (t == 0.0)
    u = 0;
  else
    u = static_cast<uint64_t>(__double_as_longlong(t));
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__global__ __launch_bounds__(kThreads) void csr_init(const double* __restrict__ time, int64_t n,
                                                     uint64_t* __restrict__ tkey,
                                                     uint32_t* __restrict__ idx) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (j >= n) return;
  tkey[j] = time_key(time[j]);
  idx[j] = static_cast<uint32_t>(j);
}

// entry j of the input: its node, neighbour, time index and event index
// (pairs: entry 2k = from[k] -> to[k], 2k + 1 = to[k] -> from[k], of event k)
struct Entries {
  const int64_t* from;
  const int64_t* to;
  const int64_t* event;
  int pairs;
  __device__ __forceinline__ int64_t node(int64_t j) const {
    return pairs ? ((j & 1) ? to[j >> 1] : from[j >> 1]) : from[j];
  }
  __device__ __forceinline__ int64_t nbr(int64_t j) const {
    return pairs ? ((j & 1) ? from[j >> 1] : to[j >> 1]) : to[j];
  }
  __device__ __forceinline__ int64_t row(int64_t j) const { return pairs ? j >> 1 : j; }
  __device__ __forceinline__ int64_t ev(int64_t j) const {
    return event != nullptr ? event[row(j)] : (pairs ? j >> 1 : -1);
  }
};

__global__ __launch_bounds__(kThreads) void csr_node_keys(Entries E,
                                                          const uint32_t* __restrict__ idx,
                                                          int64_t n, int64_t N,
                                                          uint32_t* __restrict__ nkey,
                                                          int32_t* __restrict__ status) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  bool bad = false;
  if (p < n) {
    const int64_t u = E.node(idx != nullptr ? idx[p] : p);  // NULL: the identity
    bad = u < 0 || u >= N;
    nkey[p] = bad ? 0xffffffffu : static_cast<uint32_t>(u);
  }
  const uint64_t bm = __ballot(bad);
  if ((threadIdx.x & (kWave - 1)) == 0 && bm != 0 && status != nullptr)
    atomicAdd(&status[TGX_ST_BAD_EVENT_NODE], __popcll(bm));
}

// offsets[u] = #sorted node keys < u, u in [0, N]
__global__ __launch_bounds__(kThreads) void csr_offsets(const uint32_t* __restrict__ nkey, int64_t n,
                                                        int64_t N, int64_t* __restrict__ offsets) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u > N) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(nkey[mid]) < u)
      lo = mid + 1;
    else
      hi = mid;
  }
  offsets[u] = lo;
}

// out[p] = entry perm[p]: id, time, edge id, feature row (tpe lanes per row)
template <int VEC>
__global__ __launch_bounds__(kThreads) void csr_gather(
    const uint32_t* __restrict__ perm, int64_t n, Entries E,
    const double* __restrict__ time, int64_t num_events,
    const uint8_t* __restrict__ feats, int64_t row_bytes, int tpe_log2,
    int32_t* __restrict__ out_ids, double* __restrict__ out_times, int64_t* __restrict__ out_eids,
    uint8_t* __restrict__ out_feats, int32_t* __restrict__ status) {
  using V = typename std::conditional<VEC == 16, uint4, typename std::conditional<VEC == 4, uint32_t, uint16_t>::type>::type;
  const int tpe = 1 << tpe_log2;
  const int64_t p = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> tpe_log2;
  const int l = threadIdx.x & (tpe - 1);
  bool bad = false;
  if (p < n) {
    const int64_t j = perm[p];
    const int64_t ev = E.ev(j);
    if (l == 0) {
      out_ids[p] = static_cast<int32_t>(E.nbr(j));
      out_times[p] = time[E.row(j)];
      if (out_eids != nullptr) out_eids[p] = ev;
    }
    if (out_feats != nullptr && row_bytes > 0) {
      const int nv = static_cast<int>(row_bytes / VEC);
      V* drow = reinterpret_cast<V*>(out_feats + p * row_bytes);
      const bool have = feats != nullptr && ev >= 0 && ev < num_events;
      bad = feats != nullptr && !have;
      const V* srow = have ? reinterpret_cast<const V*>(feats + ev * row_bytes) : nullptr;
      for (int c = l; c < nv; c += tpe) drow[c] = have ? srow[c] : V{};
    }
  }
  const uint64_t bm = __ballot(bad && l == 0);
  if ((threadIdx.x & (kWave - 1)) == 0 && bm != 0 && status != nullptr)
    atomicAdd(&status[TGX_ST_BAD_EVENT_NODE], __popcll(bm));
}

// Pre-freeze scan (tgx_csr_scan): node range, time order and largest time of the
// events in one pass.  Each workgroup reduces a grid-stride share into one
// ScanPart; csr_scan_final folds the parts.
constexpr int kScanParts = 1024;

struct ScanPart {
  int64_t lo, hi, bad, nd;
  double tmax;
};

// block-wide fold of (lo, hi, bad, tmax); the result is valid in thread 0
__device__ __forceinline__ ScanPart fold_block(ScanPart v, ScanPart* sm) {
  for (int o = kWave / 2; o > 0; o >>= 1) {
    v.lo = min(v.lo, static_cast<int64_t>(__shfl_xor(static_cast<long long>(v.lo), o)));
    v.hi = max(v.hi, static_cast<int64_t>(__shfl_xor(static_cast<long long>(v.hi), o)));
    v.bad += static_cast<int64_t>(__shfl_xor(static_cast<long long>(v.bad), o));
    v.nd += static_cast<int64_t>(__shfl_xor(static_cast<long long>(v.nd), o));
    v.tmax = fmax(v.tmax, __shfl_xor(v.tmax, o));
  }
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) sm[w] = v;
  __syncthreads();
  if (threadIdx.x == 0)
    for (int i = 1; i < kThreads / kWave; ++i) {
      v.lo = min(v.lo, sm[i].lo);
      v.hi = max(v.hi, sm[i].hi);
      v.bad += sm[i].bad;
      v.nd += sm[i].nd;
      v.tmax = fmax(v.tmax, sm[i].tmax);
    }
  return v;
}

// Event k >= 1 keeps the time order when t[k] - t[k-1] > 0, or == 0 with k the
// first event of an advance() call (the same float64 difference and
// comparisons as the check it replaces, so NaN and inf steps break the order).
// Every step not > 0 counts against the order, and each call start whose step
// is exactly 0 takes its count back (a second pass over the few call starts, in
// place of a search of them at every tie).  Apart, every step whose time goes
// down (or is NaN) counts against a non-decreasing stream.
__global__ __launch_bounds__(kThreads) void csr_scan_part(const int64_t* __restrict__ src,
                                                          const int64_t* __restrict__ dst,
                                                          const double* __restrict__ t, int64_t E,
                                                          const int64_t* __restrict__ starts, int64_t m,
                                                          ScanPart* __restrict__ parts) {
  __shared__ ScanPart sm[kThreads / kWave];
  ScanPart v{INT64_MAX, INT64_MIN, 0, 0, -__builtin_huge_val()};
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
#pragma unroll 4
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < E; k += stride) {
    const int64_t s = src[k], d = dst[k];
    const double x = t[k];
    v.lo = min(v.lo, min(s, d));
    v.hi = max(v.hi, max(s, d));
    if (x == x) v.tmax = fmax(v.tmax, x);
    if (k > 0) {
      const double p = t[k - 1];
      if (!(x - p > 0.0)) ++v.bad;
      if (!(x >= p)) ++v.nd;
    }
  }
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c < m; c += stride) {
    const int64_t k = starts[c];
    if (k >= 1 && k < E && (c == 0 || starts[c - 1] != k) && t[k] - t[k - 1] == 0.0) --v.bad;
  }
  v = fold_block(v, sm);
  if (threadIdx.x == 0) parts[blockIdx.x] = v;
}

// out = {min node, max node, 2 time-ordered / 1 non-decreasing / 0, bits of the largest non-NaN time}
__global__ __launch_bounds__(kThreads) void csr_scan_final(const ScanPart* __restrict__ parts, int np,
                                                           int64_t* __restrict__ out) {
  __shared__ ScanPart sm[kThreads / kWave];
  ScanPart v{INT64_MAX, INT64_MIN, 0, 0, -__builtin_huge_val()};
  for (int i = threadIdx.x; i < np; i += kThreads) {
    const ScanPart p = parts[i];
    v.lo = min(v.lo, p.lo);
    v.hi = max(v.hi, p.hi);
    v.bad += p.bad;
    v.nd += p.nd;
    v.tmax = fmax(v.tmax, p.tmax);
  }
  v = fold_block(v, sm);
  if (threadIdx.x == 0) {
    out[0] = v.lo;
    out[1] = v.hi;
    out[2] = v.bad == 0 ? 2 : (v.nd == 0 ? 1 : 0);
    out[3] = __double_as_longlong(v.tmax);
  }
}

// Build order from the events (TGX_CSR_EVENTS_BY_CALL).  The events fall into
// segments: the advance() calls, or with TGX_CSR_NONDECREASING the runs of equal
// times within a call.  The entries of segment [s, e) take build-order positions
// [2s, 2e) -- from->to of event k at s + k, then to->from at e + k -- which for
// runs of a non-decreasing stream is already its stable time order.  The
// segment of event k comes from an exclusive scan of the segment-start marks,
// so any call starts give a permutation of [0, 2E).
__global__ __launch_bounds__(kThreads) void csr_seg_marks(const double* __restrict__ time, int64_t E, int runs,
                                                          uint32_t* __restrict__ mark, uint32_t* __restrict__ ex) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (k >= E) return;
  const uint32_t f = k == 0 || (runs && !(time[k] == time[k - 1]));
  mark[k] = f;
  ex[k] = f;
}

__global__ __launch_bounds__(kThreads) void csr_seg_calls(const int64_t* __restrict__ starts, int64_t m, int64_t E,
                                                          uint32_t* __restrict__ mark, uint32_t* __restrict__ ex) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= m) return;
  const int64_t k = starts[c];
  if (k >= 1 && k < E) {
    mark[k] = 1;
    ex[k] = 1;
  }
}

// gs[segment] = its first event, gs[number of segments] = E
__global__ __launch_bounds__(kThreads) void csr_seg_starts(const uint32_t* __restrict__ mark,
                                                           const uint32_t* __restrict__ ex, int64_t E,
                                                           uint32_t* __restrict__ gs) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (k >= E) return;
  if (mark[k]) gs[ex[k]] = static_cast<uint32_t>(k);
  if (k == E - 1) gs[ex[k] + mark[k]] = static_cast<uint32_t>(E);
}

// idx[position] = entry (2k + direction); tkey (when the time passes follow) its time key
__global__ __launch_bounds__(kThreads) void csr_seg_order(const uint32_t* __restrict__ mark,
                                                          const uint32_t* __restrict__ ex,
                                                          const uint32_t* __restrict__ gs,
                                                          const double* __restrict__ time, int64_t E,
                                                          uint32_t* __restrict__ idx, uint64_t* __restrict__ tkey) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (k >= E) return;
  const uint32_t g = ex[k] + mark[k] - 1;
  const int64_t pf = static_cast<int64_t>(gs[g]) + k;
  const int64_t pr = static_cast<int64_t>(gs[g + 1]) + k;
  idx[pf] = static_cast<uint32_t>(2 * k);
  idx[pr] = static_cast<uint32_t>(2 * k + 1);
  if (tkey != nullptr) {
    const uint64_t key = time_key(time[k]);
    tkey[pf] = key;
    tkey[pr] = key;
  }
}

struct Layout {
  RadixScratch r;
  size_t tkey = 0, idx = 0, nkey = 0, count = 0, sums = 0, total = 0;
};

Layout layout(int64_t n) {
  Layout w;
  w.r = radix_scratch(n);
  const size_t un = static_cast<size_t>(std::max<int64_t>(n, 1));
  w.tkey = 0;
  w.idx = w.tkey + 2 * align256(un * 8);
  w.nkey = w.idx + 2 * align256(un * 4);
  w.count = w.nkey + 2 * align256(un * 4);
  w.sums = w.count + w.r.count_bytes;
  w.total = w.sums + w.r.sums_bytes;
  return w;
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" size_t tgx_csr_build_workspace_size(int64_t n) {
  if (n < 0) return 0;
  return layout(n).total;
}

extern "C" int tgx_csr_build(const tgx_csr_build_args* a, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (a == nullptr) return fail(TGX_ERR_ARG, "tgx_csr_build: args is NULL");
  const int64_t n = a->num_entries, N = a->num_nodes;
  if (N <= 0 || N >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "tgx_csr_build: num_nodes %lld outside [1, 2^31)", (long long)N);
  if (n < 0 || n >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "tgx_csr_build: %lld entries outside [0, 2^31)", (long long)n);
  if (a->feat_dim < 0) return fail(TGX_ERR_ARG, "tgx_csr_build: negative feat_dim");
  const int esz = feat_elem_bytes(a->feat_dtype);
  if (esz == 0) return fail(TGX_ERR_DTYPE, "tgx_csr_build: unsupported feat dtype %d", a->feat_dtype);
  if (a->out_offsets == nullptr) return fail(TGX_ERR_ARG, "tgx_csr_build: out_offsets is NULL");
  const int64_t row_bytes = static_cast<int64_t>(a->feat_dim) * esz;
  if ((a->flags & ~(TGX_CSR_EVENT_PAIRS | TGX_CSR_EVENTS_BY_CALL | TGX_CSR_NONDECREASING)) != 0)
    return fail(TGX_ERR_ARG, "tgx_csr_build: unknown flags 0x%x", a->flags);
  const int by_call = (a->flags & TGX_CSR_EVENTS_BY_CALL) != 0;
  const int runs = (a->flags & TGX_CSR_NONDECREASING) != 0;
  if ((a->flags & TGX_CSR_EVENT_PAIRS) && by_call)
    return fail(TGX_ERR_ARG, "tgx_csr_build: TGX_CSR_EVENT_PAIRS and TGX_CSR_EVENTS_BY_CALL exclude each other");
  if (runs && !by_call)
    return fail(TGX_ERR_ARG, "tgx_csr_build: TGX_CSR_NONDECREASING needs TGX_CSR_EVENTS_BY_CALL");
  if (by_call && (a->num_calls < 0 || (a->num_calls > 0 && a->call_starts == nullptr)))
    return fail(TGX_ERR_ARG, "tgx_csr_build: events by call need call_starts [num_calls >= 0]");
  // entries addressed through their events: 2k = from->to, 2k + 1 = to->from of event k
  const int pairs = (a->flags & TGX_CSR_EVENT_PAIRS) != 0 || by_call;
  if (pairs && n % 2 != 0)
    return fail(TGX_ERR_ARG, "tgx_csr_build: events need an even entry count, got %lld", (long long)n);
  if (n > 0) {
    if (a->from == nullptr || a->to == nullptr || a->time == nullptr || a->out_ids == nullptr ||
        a->out_times == nullptr)
      return fail(TGX_ERR_ARG, "tgx_csr_build: from/to/time/out_ids/out_times must not be NULL");
    if (row_bytes > 0 && a->out_feats == nullptr)
      return fail(TGX_ERR_ARG, "tgx_csr_build: out_feats is NULL with feat_dim > 0");
    if ((a->feats != nullptr || a->out_eids != nullptr) && a->event == nullptr && !pairs)
      return fail(TGX_ERR_ARG, "tgx_csr_build: feats / out_eids need the event index array");
    if (a->feats != nullptr && a->num_events < 0)
      return fail(TGX_ERR_ARG, "tgx_csr_build: negative num_events");
  }
  const Layout w = layout(n);
  if (a->workspace == nullptr || a->workspace_bytes < w.total)
    return fail(TGX_ERR_ARG, "tgx_csr_build: workspace of %zu bytes needed, got %zu", w.total,
                a->workspace_bytes);
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  const unsigned g1 = static_cast<unsigned>(std::max<int64_t>(cdiv(n, kThreads), 1));
  int rc;
  if (n == 0) {
    hipLaunchKernelGGL(csr_offsets, dim3(static_cast<unsigned>(cdiv(N + 1, kThreads))), dim3(kThreads),
                       0, stream, static_cast<const uint32_t*>(nullptr), n, N, a->out_offsets);
    return check_launch("csr_offsets");
  }
  const size_t un = static_cast<size_t>(n);
  uint64_t* tk[2] = {reinterpret_cast<uint64_t*>(ws + w.tkey),
                     reinterpret_cast<uint64_t*>(ws + w.tkey + align256(un * 8))};
  uint32_t* ix[2] = {reinterpret_cast<uint32_t*>(ws + w.idx),
                     reinterpret_cast<uint32_t*>(ws + w.idx + align256(un * 4))};
  uint32_t* nk[2] = {reinterpret_cast<uint32_t*>(ws + w.nkey),
                     reinterpret_cast<uint32_t*>(ws + w.nkey + align256(un * 4))};
  uint32_t* count = reinterpret_cast<uint32_t*>(ws + w.count);
  uint32_t* sums = reinterpret_cast<uint32_t*>(ws + w.sums);
  const Entries E{a->from, a->to, a->event, pairs};
  int cur = 0;
  if (by_call) {
    // the build order from the segments; marks and their scan in nk[0], the
    // segment starts in nk[1], the scan's tile sums in the digit counts (free
    // until the first pass)
    const int64_t ne = n / 2;
    const unsigned ge = static_cast<unsigned>(cdiv(ne, kThreads));
    uint32_t* mark = nk[0];
    uint32_t* ex = nk[0] + ne;
    hipLaunchKernelGGL(csr_seg_marks, dim3(ge), dim3(kThreads), 0, stream, a->time, ne, runs, mark, ex);
    if ((rc = check_launch("csr_seg_marks"))) return rc;
    if (a->num_calls > 0) {
      hipLaunchKernelGGL(csr_seg_calls, dim3(static_cast<unsigned>(cdiv(a->num_calls, kThreads))), dim3(kThreads), 0,
                         stream, a->call_starts, a->num_calls, ne, mark, ex);
      if ((rc = check_launch("csr_seg_calls"))) return rc;
    }
    if ((rc = scan_exclusive(ex, ne, count, scan_levels(ne), 0, stream))) return rc;
    hipLaunchKernelGGL(csr_seg_starts, dim3(ge), dim3(kThreads), 0, stream, static_cast<const uint32_t*>(mark),
                       static_cast<const uint32_t*>(ex), ne, nk[1]);
    if ((rc = check_launch("csr_seg_starts"))) return rc;
    hipLaunchKernelGGL(csr_seg_order, dim3(ge), dim3(kThreads), 0, stream, static_cast<const uint32_t*>(mark),
                       static_cast<const uint32_t*>(ex), static_cast<const uint32_t*>(nk[1]), a->time, ne, ix[0],
                       runs ? static_cast<uint64_t*>(nullptr) : tk[0]);
    if ((rc = check_launch("csr_seg_order"))) return rc;
    // stable by time unless the runs already are
    if (!runs && (rc = radix_sort<uint64_t>(tk, ix, cur, n, 64, w.r, count, sums, stream))) return rc;
  } else if (pairs) {
    // already in stable time order: the identity, which the node keys and the
    // first node pass take without reading it
  } else {
    hipLaunchKernelGGL(csr_init, dim3(g1), dim3(kThreads), 0, stream, a->time, n, tk[0], ix[0]);
    if ((rc = check_launch("csr_init"))) return rc;
    // stable by time: 8 passes, ping-pong ending in buffer 0
    if ((rc = radix_sort<uint64_t>(tk, ix, cur, n, 64, w.r, count, sums, stream))) return rc;
  }
  // then stable by node over ceil(log2 N) bits (out-of-range ids sort last)
  const bool ident = pairs && !by_call;
  hipLaunchKernelGGL(csr_node_keys, dim3(g1), dim3(kThreads), 0, stream, E,
                     ident ? static_cast<const uint32_t*>(nullptr) : static_cast<const uint32_t*>(ix[cur]), n, N,
                     nk[0], a->status);
  if ((rc = check_launch("csr_node_keys"))) return rc;
  int bits = 1;
  while ((int64_t(1) << bits) < N + 1) ++bits;  // + 1: the out-of-range key 0xffffffff
  // the node keys ride in nk[], the permutation in ix[] (starting where the time
  // passes left it)
  uint32_t* pv[2] = {ix[cur], ix[1 - cur]};
  int ncur = 0;
  if ((rc = radix_sort<uint32_t>(nk, pv, ncur, n, bits, w.r, count, sums, stream, ident))) return rc;
  uint32_t* perm_in = pv[ncur];
  hipLaunchKernelGGL(csr_offsets, dim3(static_cast<unsigned>(cdiv(N + 1, kThreads))), dim3(kThreads), 0,
                     stream, static_cast<const uint32_t*>(nk[ncur]), n, N, a->out_offsets);
  if ((rc = check_launch("csr_offsets"))) return rc;
  int vec = 2;
  const bool fe = row_bytes > 0;
  auto al = [](const void* p, unsigned m) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & m) == 0; };
  if (row_bytes % 16 == 0 && (!fe || (al(a->feats, 15) && al(a->out_feats, 15))))
    vec = 16;
  else if (row_bytes % 4 == 0 && (!fe || (al(a->feats, 3) && al(a->out_feats, 3))))
    vec = 4;
  const int64_t nchunks = fe ? row_bytes / vec : 1;
  int tpe_log2 = 0;
  while ((int64_t(1) << tpe_log2) < nchunks && tpe_log2 < 6) ++tpe_log2;
  const dim3 gg(static_cast<unsigned>(cdiv(n << tpe_log2, kThreads)));
  auto gather = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, gg, dim3(kThreads), 0, stream, static_cast<const uint32_t*>(perm_in), n,
                       E, a->time, a->num_events,
                       static_cast<const uint8_t*>(a->feats), fe ? row_bytes : 0, tpe_log2, a->out_ids,
                       a->out_times, a->out_eids, static_cast<uint8_t*>(fe ? a->out_feats : nullptr),
                       a->status);
  };
  if (vec == 16)
    gather(csr_gather<16>);
  else if (vec == 4)
    gather(csr_gather<4>);
  else
    gather(csr_gather<2>);
  return check_launch("csr_gather");
}

extern "C" size_t tgx_csr_scan_workspace_size(void) { return kScanParts * sizeof(ScanPart); }

extern "C" int tgx_csr_scan(const int64_t* src, const int64_t* dst, const double* time, int64_t num_events,
                            const int64_t* call_starts, int64_t num_calls, int64_t* out, void* workspace,
                            size_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (num_events <= 0) return fail(TGX_ERR_ARG, "tgx_csr_scan: num_events %lld must be positive", (long long)num_events);
  if (num_calls < 0) return fail(TGX_ERR_ARG, "tgx_csr_scan: negative num_calls");
  if (src == nullptr || dst == nullptr || time == nullptr || out == nullptr ||
      (num_calls > 0 && call_starts == nullptr))
    return fail(TGX_ERR_ARG, "tgx_csr_scan: src/dst/time/out (and call_starts when num_calls > 0) must not be NULL");
  if (workspace == nullptr || workspace_bytes < tgx_csr_scan_workspace_size())
    return fail(TGX_ERR_ARG, "tgx_csr_scan: workspace of %zu bytes needed, got %zu", tgx_csr_scan_workspace_size(),
                workspace_bytes);
  // about four events per thread before the grid reaches kScanParts workgroups
  const int np = static_cast<int>(std::min<int64_t>(cdiv(num_events, 4 * kThreads), kScanParts));
  ScanPart* parts = static_cast<ScanPart*>(workspace);
  hipLaunchKernelGGL(csr_scan_part, dim3(np), dim3(kThreads), 0, stream, src, dst, time, num_events, call_starts,
                     num_calls, parts);
  int rc;
  if ((rc = check_launch("csr_scan_part"))) return rc;
  hipLaunchKernelGGL(csr_scan_final, dim3(1), dim3(kThreads), 0, stream, static_cast<const ScanPart*>(parts), np,
                     out);
  return check_launch("csr_scan_final");
}
