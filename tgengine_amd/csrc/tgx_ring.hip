// Kernel (a): ring-buffer update for one batch of events.
//
// Semantics (reference tgengine/core/temporal_graph.py:123-129 and
// _append_overflow :351-387): the batch of b undirected events becomes n = 2b
// directed entries in concatenation order i = [src->dst for every event,
// dst->src for every event].  Grouped by `from` node in that order, each node
// with c entries keeps its last min(c, B); the m-th kept entry goes to slot
// (write_pos + m) % B and write_pos grows by min(c, B).  Equivalently, the
// entry with e later same-node entries is kept iff e < kept = min(c, B) and
// lands in slot (write_pos + kept - 1 - e) % B.
//
// Batches of up to kFastMaxEntries entries: two launches.
//   plan   : every entry's rank among its node's entries in entry order, from
//            its workgroup's scan of the batch's node ids (entries of its nodes
//            before and after its range) and wavefront ballots over its own
//            range (tgx_ring_plan.h); the entry's record holds its ring slot if
//            it is kept (rank >= c - kept) and, on the node's last entry, the
//            node's new write position.  No workgroup waits for another.
//   commit : one copy per entry: the record, node, neighbour, time and row in
//            one round trip, then the kept entries' stores.
// Larger batches: four launches, with per-node tickets from node-indexed
// counters owned by the ring (zero between calls; equal nodes of a workgroup
// are first aggregated in an LDS hash table, so a node costs one global atomic
// per workgroup however hot it is) and lists sized after counting.
//   count  : tickets, in no particular order.
//   groups : the ticket-0 entry of every node seen more than once reserves
//            a contiguous list of c slots and a group id, small (c <= 64)
//            or large (one atomic per wave, offsets by a wave scan).
//   fill   : list[base[u] + ticket] = entry index.
//   commit : singletons (c == 1) are written directly; a small group is ranked
//            by one wavefront in registers, a large group by a whole workgroup
//            over bitmap windows walked down from the top of the batch; the
//            counters are restored to zero.
// Every path writes the kept entries and advances write_pos.  Feature rows move
// as 16-byte vectors when the row allows it.
#include "tgx_ring_plan.h"

#include <algorithm>
#include <mutex>

namespace tgx {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kCommitWaves = kThreads / kWave;
constexpr int kWinBits = 8192;                 // bitmap window (indices)
constexpr int kWinWords = kWinBits / 32;       // 256 words = 1 KB
static_assert(kWinWords == kThreads, "one bitmap word per thread");
constexpr int64_t kSmallGroupBlocks = 256;  // commit blocks for small groups (4 waves each)
constexpr int64_t kLargeGroupBlocks = 64;   // four-launch commit blocks for large groups

// (write_pos + off) % B for write_pos >= 0, 0 <= off < B
__device__ __forceinline__ int64_t ring_slot(int64_t w, int off, int B) {
  const uint64_t x = static_cast<uint64_t>(w) + static_cast<uint64_t>(off);
  if ((B & (B - 1)) == 0) return static_cast<int64_t>(x & static_cast<uint64_t>(B - 1));
  if (x < (uint64_t(1) << 32))
    return static_cast<int64_t>(static_cast<uint32_t>(x) % static_cast<uint32_t>(B));
  return static_cast<int64_t>(x % static_cast<uint64_t>(B));
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

struct AppendParams : PlanParams {
  const uint8_t* feat;  // [b, row_bytes] or null (zero rows)
  int B;
  int64_t row_bytes;
  int64_t eid_base;
  int32_t* ids;
  double* times;
  uint8_t* feats;
  int64_t* wp;
  int64_t* eids;
  int32_t* nbase;   // [N] four-launch list base of multi-entry nodes (over lst)
  int32_t* status;
  int tpe_log2;     // lanes per entry (kept_commit, four-launch singletons)
  int ga;           // four-launch commit: blocks of the singleton role
  int gb;           // four-launch commit: blocks of the small-group role
};

// the plan's diagnostics (words time_word, bad_word) reach the status words only
// when the batch commits
__device__ __forceinline__ void commit_diagnostics(const AppendParams& P, int time_word, int bad_word) {
  if (P.status != nullptr) {
    if (P.ctl[bad_word] != 0) atomicAdd(&P.status[TGX_ST_BAD_EVENT_NODE], P.ctl[bad_word]);
    if (P.ctl[time_word] == 0) atomicAdd(&P.status[TGX_ST_KEY_COLLISION], 1);
  }
  P.ctl[time_word] = 0;
  P.ctl[bad_word] = 0;
}

// ---- four-launch 1. count ----------------------------------------------------
__global__ __launch_bounds__(kThreads) void append_count(PlanParams P) {
  __shared__ PlanLds L;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i == 0) {
    P.ctl[kCtlCursor] = 0;
    P.ctl[kCtlGroups] = 0;
    P.ctl[kCtlLarge] = 0;
  }
  int bad;
  bool time_ok;
  const int32_t u = entry_prologue(P, i, bad, time_ok);
  const int32_t t = node_ticket(P, u, L);
  if (i < P.n) P.ticket[i] = t;
  report_diagnostics(P, bad, time_ok, kCtlTimeOk, kCtlBad);
}

// ---- two-launch 1. plan -------------------------------------------------------
// Alone, the plan's workgroups are as large as they go: each scans the whole
// batch, so T threads take n/T node ids each, all loaded in one or two steps.
constexpr int kPlanAloneThreads = 1024;
constexpr int kPlanAloneScan = 8;
template <int T>
__global__ __launch_bounds__(T) void fast_plan(PlanParams P) {
  __shared__ __align__(16) uint8_t smem[plan_lds_bytes(T)];
  plan_block_ordered<T == kPlanAloneThreads ? kPlanAloneScan : 4>(P, blockIdx.x, smem);
}

// ---- four-launch 2. groups --------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void append_groups(AppendParams P) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  int64_t u = -1;
  int c = 0;
  if (i < P.n && P.ticket[i] == 0) {
    u = entry_node(P.src, P.dst, i, P.b);
    c = P.cnt[u];
  }
  const bool grp = c > 1;
  const bool big = c > kWave;
  // wave-aggregated reservation of group ids and list space
  const uint64_t sm = __ballot(grp && !big);
  const uint64_t lm = __ballot(big);
  const int sum = grp ? c : 0;
  int incl = sum;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += y;
  }
  const int total = __shfl(incl, kWave - 1, kWave);
  int sbase = 0, lgbase = 0, lbase = 0;
  if ((sm | lm) != 0) {
    if (lane == 0) {
      if (sm) sbase = atomicAdd(&P.ctl[kCtlGroups], __popcll(sm));
      if (lm) lgbase = atomicAdd(&P.ctl[kCtlLarge], __popcll(lm));
      lbase = atomicAdd(&P.ctl[kCtlCursor], total);
    }
    sbase = __shfl(sbase, 0, kWave);
    lgbase = __shfl(lgbase, 0, kWave);
    lbase = __shfl(lbase, 0, kWave);
  }
  const uint64_t below = (uint64_t(1) << lane) - 1;
  if (grp && !big) P.groups[sbase + __popcll(sm & below)] = static_cast<int32_t>(u);
  if (big) P.large[lgbase + __popcll(lm & below)] = static_cast<int32_t>(u);
  if (grp) P.nbase[u] = lbase + incl - sum;
}

// ---- four-launch 3. fill ----------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void append_fill(AppendParams P) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= P.n) return;
  const int t = P.ticket[i];
  if (t < 0) return;
  const int64_t u = entry_node(P.src, P.dst, i, P.b);
  if (P.cnt[u] > 1) P.list[P.nbase[u] + t] = static_cast<int32_t>(i);
}

// write id / time / edge id of entry i into ring slot `slot` (global index)
__device__ __forceinline__ void write_entry_meta(const AppendParams& P, int64_t i, int64_t slot) {
  const int64_t e = i < P.b ? i : i - P.b;
  P.ids[slot] = static_cast<int32_t>(i < P.b ? P.dst[e] : P.src[e]);
  P.times[slot] = P.time[e];
  if (P.eids != nullptr) P.eids[slot] = P.eid_base + e;
}

// row chunks each thread loads before storing them when it copies kept rows
constexpr int kKeptDepth = 4;

// copy the kept rows R[0..kept) of node u (row r -> slot (w + kept - 1 - r) % B);
// threads t = first, first + stride, ... of the caller share the work.  Loads
// and stores share one in-order vmcnt, so every load of a round (the thread's
// first row's id and time, kKeptDepth row chunks) is issued before its stores:
// a row of many chunks costs one round trip per kKeptDepth chunks, not per chunk.
template <int VEC>
__device__ __forceinline__ void write_kept(const AppendParams& P, const int32_t* R, int64_t u,
                                           int kept, int64_t w, int first, int stride) {
  using V = typename VecT<VEC>::T;
  const int nv = static_cast<int>(P.row_bytes / VEC);
  const int total = kept * nv;
  // the thread's first row: id, time, edge id (loaded with the first chunks)
  int32_t m_id = 0;
  double m_t = 0.0;
  int64_t m_slot = -1, m_e = 0;
  if (first < kept) {
    const int64_t i = R[first];
    m_e = i < P.b ? i : i - P.b;
    m_id = static_cast<int32_t>(i < P.b ? P.dst[m_e] : P.src[m_e]);
    m_t = P.time[m_e];
    m_slot = u * P.B + ring_slot(w, kept - 1 - first, P.B);
  }
  for (int f0 = first; f0 < total || m_slot >= 0; f0 += kKeptDepth * stride) {
    V v[kKeptDepth];
    V* dp[kKeptDepth];
#pragma unroll
    for (int k = 0; k < kKeptDepth; ++k) {
      const int f = f0 + k * stride;
      dp[k] = nullptr;
      v[k] = V{};
      if (f < total) {
        const int r = f / nv;
        const int cch = f - r * nv;
        const int64_t i = R[r];
        const int64_t e = i < P.b ? i : i - P.b;
        const int64_t slot = u * P.B + ring_slot(w, kept - 1 - r, P.B);
        dp[k] = reinterpret_cast<V*>(P.feats + slot * P.row_bytes) + cch;
        if (P.feat != nullptr) v[k] = reinterpret_cast<const V*>(P.feat + e * P.row_bytes)[cch];
      }
    }
    if (m_slot >= 0) {
      P.ids[m_slot] = m_id;
      P.times[m_slot] = m_t;
      if (P.eids != nullptr) P.eids[m_slot] = P.eid_base + m_e;
      m_slot = -1;
    }
#pragma unroll
    for (int k = 0; k < kKeptDepth; ++k)
      if (dp[k] != nullptr) *dp[k] = v[k];
  }
  // rows beyond the first of this thread (only when kept > stride)
  for (int r = first + stride; r < kept; r += stride)
    write_entry_meta(P, R[r], u * P.B + ring_slot(w, kept - 1 - r, P.B));
}

// one large group (c > 64) by the whole workgroup
template <int VEC>
__device__ __forceinline__ void commit_large(const AppendParams& P, int64_t gid, uint32_t* bitmap,
                                             int32_t* sfx, int32_t* R, int32_t* wsum) {
  const int wv = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int t = threadIdx.x;
  const int64_t u = P.large[gid];
  const int c = P.cnt[u];
  const int base = P.nbase[u];
  const int kept = c < P.B ? c : P.B;
  int64_t hi = P.n;
  int carry = 0;
  while (carry < kept && hi > 0) {  // uniform across the workgroup
    const int64_t lo = hi > kWinBits ? hi - kWinBits : 0;
    for (int q = t; q < kWinWords; q += kThreads) bitmap[q] = 0u;
    __syncthreads();
    for (int j = t; j < c; j += kThreads) {
      const int64_t x = P.list[base + j];
      if (x >= lo && x < hi) atomicOr(&bitmap[(x - lo) >> 5], 1u << ((x - lo) & 31));
    }
    __syncthreads();
    // exclusive suffix over words: thread t owns word t (kWinWords == kThreads)
    const int own = __popc(bitmap[t]);
    int suf = own;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int y = __shfl_down(suf, off, kWave);
      if (lane + off < kWave) suf += y;
    }
    if (lane == 0) wsum[wv] = suf;
    __syncthreads();
    int later = 0, win_total = 0;
    for (int w2 = 0; w2 < kCommitWaves; ++w2) {
      if (w2 > wv) later += wsum[w2];
      win_total += wsum[w2];
    }
    sfx[t] = later + suf - own;
    __syncthreads();
    for (int j = t; j < c; j += kThreads) {
      const int64_t x = P.list[base + j];
      if (x >= lo && x < hi) {
        const int rel = static_cast<int>(x - lo);
        const int word = rel >> 5;
        const int e = carry + (__popc(bitmap[word] >> (rel & 31)) - 1) + sfx[word];
        if (e < kept) R[e] = static_cast<int32_t>(x);
      }
    }
    carry += win_total;
    hi = lo;
    __syncthreads();
  }
  const int64_t w = P.wp[u];
  write_kept<VEC>(P, R, u, kept, w, t, kThreads);
  __syncthreads();
  if (t == 0) {
    P.wp[u] = w + kept;
    P.cnt[u] = 0;
  }
  __syncthreads();  // the next group rewrites R and the bitmap
}

// singletons (c == 1), written directly: tpe lanes per entry, blocks [0, ga).
// A group's counter reads c >= 2 or 0 (once its role restored it), never 1.
// Each lane holds up to kKeptDepth chunks of the row (tpe <= 16 lanes per entry,
// so 16-byte chunks cover rows up to 1 KB in one round); longer rows continue
// in rounds of kKeptDepth loads, then stores.
template <int VEC>
__device__ __forceinline__ void commit_singletons(const AppendParams& P, int blk) {
  using V = typename VecT<VEC>::T;
  const int nv = static_cast<int>(P.row_bytes / VEC);
  const int tpe = 1 << P.tpe_log2;
  const int epb = static_cast<int>(blockDim.x) >> P.tpe_log2;
  const int64_t i = static_cast<int64_t>(blk) * epb + (threadIdx.x >> P.tpe_log2);
  const int l = threadIdx.x & (tpe - 1);
  if (i >= P.n) return;
  // the entry's own data is read with its node, before the node is known to be
  // a singleton, so the role costs two round trips
  const int64_t e = i < P.b ? i : i - P.b;
  const int64_t u = entry_node(P.src, P.dst, i, P.b);
  const V* srow = reinterpret_cast<const V*>(P.feat + e * P.row_bytes);
  V v[kKeptDepth];
#pragma unroll
  for (int k = 0; k < kKeptDepth; ++k) {
    const int c = l + k * tpe;
    v[k] = (P.feat != nullptr && c < nv) ? srow[c] : V{};
  }
  int32_t other = 0;
  double tm = 0.0;
  if (l == 0) {
    other = static_cast<int32_t>(i < P.b ? P.dst[e] : P.src[e]);
    tm = P.time[e];
  }
  if (u < 0 || u >= P.N) return;
  // the counter and the write position in one round trip
  const int32_t cn = P.cnt[u];
  const int64_t w = P.wp[u];
  if (cn != 1) return;
  const int64_t slot = u * P.B + ring_slot(w, 0, P.B);
  V* drow = reinterpret_cast<V*>(P.feats + slot * P.row_bytes);
#pragma unroll
  for (int k = 0; k < kKeptDepth; ++k) {
    const int c = l + k * tpe;
    if (c < nv) drow[c] = v[k];
  }
  for (int c0 = l + kKeptDepth * tpe; c0 < nv; c0 += kKeptDepth * tpe) {
#pragma unroll
    for (int k = 0; k < kKeptDepth; ++k) {
      const int c = c0 + k * tpe;
      v[k] = (P.feat != nullptr && c < nv) ? srow[c] : V{};
    }
#pragma unroll
    for (int k = 0; k < kKeptDepth; ++k) {
      const int c = c0 + k * tpe;
      if (c < nv) drow[c] = v[k];
    }
  }
  if (l == 0) {
    P.ids[slot] = other;
    P.times[slot] = tm;
    if (P.eids != nullptr) P.eids[slot] = P.eid_base + e;
    P.wp[u] = w + 1;
    P.cnt[u] = 0;
  }
}

// one group of c <= kWave entries listed in idx (lane j < c holds one entry
// index), ranked in registers by one wavefront, then written
template <int VEC>
__device__ __forceinline__ void commit_small(const AppendParams& P, int64_t u, int c, int32_t idx,
                                             int64_t w, int32_t* R) {
  const int lane = threadIdx.x & (kWave - 1);
  const int kept = c < P.B ? c : P.B;
  int e = 0;
  for (int j = 0; j < c; ++j) e += __shfl(idx, j, kWave) > idx;
  if (lane < c && e < kept) R[e] = idx;
  wave_sync_lds();
  write_kept<VEC>(P, R, u, kept, w, lane, kWave);
  if (lane == 0) {
    P.wp[u] = w + kept;
    P.cnt[u] = 0;
  }
  wave_sync_lds();  // R is rewritten by the next group
}

// ---- four-launch 4. commit ----------------------------------------------------
// blocks [0, ga): singletons; [ga, ga+gb): small groups, one per wavefront;
// [ga+gb, ...): large groups, one per workgroup
template <int VEC>
__global__ __launch_bounds__(kThreads) void append_commit(AppendParams P) {
  __shared__ uint32_t bitmap[kWinWords];
  __shared__ int32_t sfx[kWinWords];                     // set bits in later words
  __shared__ int32_t rows[kCommitWaves][TGX_MAX_SLOTS];  // kept entry index by e
  __shared__ int32_t wsum[kCommitWaves];
  const int blk = static_cast<int>(blockIdx.x);
  if (blk == 0 && threadIdx.x == 0) commit_diagnostics(P, kCtlTimeOk, kCtlBad);
  if (blk < P.ga) {
    commit_singletons<VEC>(P, blk);
    return;
  }
  const int wv = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (blk < P.ga + P.gb) {
    // small groups (2 <= c <= 64), one per wavefront, strided over the gb blocks
    const int64_t ngroups = P.ctl[kCtlGroups];
    for (int64_t gid = static_cast<int64_t>(blk - P.ga) * kCommitWaves + wv; gid < ngroups;
         gid += static_cast<int64_t>(P.gb) * kCommitWaves) {  // wave-uniform
      const int64_t u = P.groups[gid];
      const int c = P.cnt[u];
      const int32_t idx = lane < c ? P.list[P.nbase[u] + lane] : -1;
      commit_small<VEC>(P, u, c, idx, P.wp[u], rows[wv]);
    }
    return;
  }
  // large groups (c > 64), one per workgroup, strided over the remaining blocks:
  // the workgroup ranks the list over bitmap windows of kWinBits entry indices,
  // from the top of the batch down, until `kept` entries are found
  const int64_t nlarge = P.ctl[kCtlLarge];
  const int64_t gstride = static_cast<int64_t>(gridDim.x) - P.ga - P.gb;
  for (int64_t gid = blk - P.ga - P.gb; gid < nlarge; gid += gstride)  // workgroup-uniform
    commit_large<VEC>(P, gid, bitmap, sfx, rows[0], wsum);
}

// ---- two-launch 2. commit -------------------------------------------------------
// One entry per tpe lanes (one 16-byte chunk of its row each, as the four-launch
// singletons): the plan's record of the entry (its ring slot or -1, and the
// node's new write position on the node's last entry), the entry's node,
// neighbour, time and feature row arrive in one round trip; a kept entry is
// written to its slot.  Rows longer than kKeptDepth chunks per lane continue in
// rounds of kKeptDepth loads, then stores.  Workgroup 0 reports and clears the
// plan's diagnostics.
constexpr int kKeptThreads = 256;
template <int VEC>
__global__ __launch_bounds__(kKeptThreads) void kept_commit(AppendParams P) {
  using V = typename VecT<VEC>::T;
  if (blockIdx.x == 0 && threadIdx.x == 0) commit_diagnostics(P, kCtlKTime, kCtlKBad);
  const int nv = static_cast<int>(P.row_bytes / VEC);
  const int tpe = 1 << P.tpe_log2;
  const int epb = kKeptThreads >> P.tpe_log2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * epb + (threadIdx.x >> P.tpe_log2);
  const int l = threadIdx.x & (tpe - 1);
  if (i >= P.n) return;
  const longlong2 kr = reinterpret_cast<const longlong2*>(P.krec)[i];
  const int64_t e = i < P.b ? i : i - P.b;
  const int64_t u = entry_node(P.src, P.dst, i, P.b);
  const V* srow = reinterpret_cast<const V*>(P.feat + e * P.row_bytes);
  V v[kKeptDepth];
#pragma unroll
  for (int k = 0; k < kKeptDepth; ++k) {
    const int c = l + k * tpe;
    v[k] = (P.feat != nullptr && c < nv) ? srow[c] : V{};
  }
  int32_t other = 0;
  double tm = 0.0;
  if (l == 0) {
    other = static_cast<int32_t>(i < P.b ? P.dst[e] : P.src[e]);
    tm = P.time[e];
  }
  if (kr.x >= 0) {
    const int64_t slot = u * P.B + kr.x;
    V* drow = reinterpret_cast<V*>(P.feats + slot * P.row_bytes);
#pragma unroll
    for (int k = 0; k < kKeptDepth; ++k) {
      const int c = l + k * tpe;
      if (c < nv) drow[c] = v[k];
    }
    for (int c0 = l + kKeptDepth * tpe; c0 < nv; c0 += kKeptDepth * tpe) {
#pragma unroll
      for (int k = 0; k < kKeptDepth; ++k) {
        const int c = c0 + k * tpe;
        v[k] = (P.feat != nullptr && c < nv) ? srow[c] : V{};
      }
#pragma unroll
      for (int k = 0; k < kKeptDepth; ++k) {
        const int c = c0 + k * tpe;
        if (c < nv) drow[c] = v[k];
      }
    }
    if (l == 0) {
      P.ids[slot] = other;
      P.times[slot] = tm;
      if (P.eids != nullptr) P.eids[slot] = P.eid_base + e;
    }
  }
  if (l == 0 && kr.y >= 0) P.wp[u] = kr.y;
}

// ---- discard: restore the scratch of a planned batch without committing it ----
__global__ __launch_bounds__(kThreads) void append_discard(PlanParams P, int two_launch) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i == 0) {
    P.ctl[two_launch ? kCtlKTime : kCtlTimeOk] = 0;
    P.ctl[two_launch ? kCtlKBad : kCtlBad] = 0;
  }
  // a two-launch plan leaves no per-node state
  if (two_launch || i >= P.n) return;
  const int64_t u = entry_node(P.src, P.dst, i, P.b);
  if (u >= 0 && u < P.N) P.cnt[u] = 0;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" size_t tgx_ring_append_workspace_size(int64_t b) {
  if (b <= 0) return 256;
  const size_t n = static_cast<size_t>(2 * b);
  // four-launch: ticket | lists | groups | large; two-launch (n <= kFastMaxEntries):
  // and the plan's entry records
  return align256(n * 4) + align256(n * 4) + align256((n / 2 + 1) * 4) +
         align256((n / (kListCap + 1) + 1) * 4) +
         (n <= static_cast<size_t>(kFastMaxEntries) ? align256(n * 16) : 0);
}

extern "C" size_t tgx_ring_scratch_size(int64_t num_nodes) {
  if (num_nodes < 0) return 0;
  return static_cast<size_t>(ctl_offset(num_nodes) + kCtlWords) * sizeof(int32_t);
}

namespace tgx {

int plan_setup(const char* who, const tgx_ring* ring, const int64_t* src, const int64_t* dst,
               const double* time, int64_t b, void* workspace, size_t workspace_bytes,
               PlanParams& P) {
  P = PlanParams{};
  if (ring == nullptr) return fail(TGX_ERR_ARG, "%s: ring is NULL", who);
  if (b < 0) return fail(TGX_ERR_ARG, "%s: negative batch size %lld", who, (long long)b);
  if (b == 0) return TGX_OK;
  if (src == nullptr || dst == nullptr || time == nullptr)
    return fail(TGX_ERR_ARG, "%s: src/dst/time must not be NULL", who);
  if (ring->scratch == nullptr) return fail(TGX_ERR_ARG, "%s: ring scratch must not be NULL", who);
  if (ring->num_nodes <= 0 || ring->num_nodes >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "%s: num_nodes %lld outside [1, 2^31)", who, (long long)ring->num_nodes);
  const int64_t n = 2 * b;
  if (n >= (int64_t(1) << 30)) return fail(TGX_ERR_LIMIT, "%s: batch too large", who);
  const size_t need = tgx_ring_append_workspace_size(b);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(TGX_ERR_ARG, "%s: workspace of %zu bytes needed, got %zu", who, need, workspace_bytes);
  if (!aligned16(workspace))
    return fail(TGX_ERR_ARG, "%s: workspace must be 16-byte aligned", who);
  P.src = src;
  P.dst = dst;
  P.time = time;
  P.b = b;
  P.n = n;
  P.N = ring->num_nodes;
  P.cnt = ring->scratch;
  P.lst = ring->scratch + ring->num_nodes;
  P.ctl = ring->scratch + ctl_offset(ring->num_nodes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const size_t o_list = align256(static_cast<size_t>(n) * 4);
  const size_t o_groups = o_list + align256(static_cast<size_t>(n) * 4);
  P.ticket = reinterpret_cast<int32_t*>(ws);
  P.list = reinterpret_cast<int32_t*>(ws + o_list);
  P.groups = reinterpret_cast<int32_t*>(ws + o_groups);
  const size_t o_large = o_groups + align256(static_cast<size_t>(n / 2 + 1) * 4);
  P.large = reinterpret_cast<int32_t*>(ws + o_large);
  P.krec = n <= kFastMaxEntries
               ? reinterpret_cast<int64_t*>(ws + o_large + align256(static_cast<size_t>(n / (kListCap + 1) + 1) * 4))
               : nullptr;
  P.wpos = ring->write_pos;
  P.B = ring->slots;
  return TGX_OK;
}

int launch_plan(const PlanParams& P, hipStream_t stream) {
  const dim3 grid1(static_cast<unsigned>((P.n + kThreads - 1) / kThreads));
  if (plan_fused_ok(P)) {
    if (P.n <= kThreads) {
      hipLaunchKernelGGL(fast_plan<kThreads>, grid1, dim3(kThreads), 0, stream, P);
    } else {
      const dim3 grid(static_cast<unsigned>((P.n + kPlanAloneThreads - 1) / kPlanAloneThreads));
      hipLaunchKernelGGL(fast_plan<kPlanAloneThreads>, grid, dim3(kPlanAloneThreads), 0, stream, P);
    }
    return check_launch("fast_plan");
  }
  // the four-launch plan: groups and fill also read the lists' aliases
  AppendParams A{};
  static_cast<PlanParams&>(A) = P;
  A.nbase = P.lst;
  hipLaunchKernelGGL(append_count, grid1, dim3(kThreads), 0, stream, static_cast<const PlanParams&>(A));
  int rc = check_launch("append_count");
  if (rc) return rc;
  hipLaunchKernelGGL(append_groups, grid1, dim3(kThreads), 0, stream, A);
  if ((rc = check_launch("append_groups"))) return rc;
  hipLaunchKernelGGL(append_fill, grid1, dim3(kThreads), 0, stream, A);
  return check_launch("append_fill");
}

namespace {

// argument checks and the kernel parameters shared by append / commit
int setup_append(const char* who, const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                 const double* time, const void* feat, int64_t b, int64_t eid_base, void* workspace,
                 size_t workspace_bytes, int32_t* status, AppendParams& P, int& vec) {
  P = AppendParams{};
  int rc = plan_setup(who, ring, src, dst, time, b, workspace, workspace_bytes, P);
  if (rc != TGX_OK || b == 0) return rc;
  if (ring->ids == nullptr || ring->times == nullptr || ring->write_pos == nullptr ||
      (ring->feats == nullptr && ring->feat_dim > 0))
    return fail(TGX_ERR_ARG, "%s: ring arrays (ids, times, feats, write_pos) must not be NULL", who);
  const int esz = feat_elem_bytes(ring->feat_dtype);
  if (esz == 0) return fail(TGX_ERR_DTYPE, "%s: unsupported feat dtype %d", who, ring->feat_dtype);
  if (ring->slots < 1 || ring->slots > TGX_MAX_SLOTS)
    return fail(TGX_ERR_LIMIT, "%s: slots %d outside [1, %d]", who, ring->slots, TGX_MAX_SLOTS);
  if (ring->feat_dim < 0) return fail(TGX_ERR_ARG, "%s: negative feat_dim", who);
  const int64_t n = P.n;
  P.feat = static_cast<const uint8_t*>(feat);
  P.B = ring->slots;
  P.row_bytes = static_cast<int64_t>(ring->feat_dim) * esz;
  P.eid_base = eid_base;
  P.ids = ring->ids;
  P.times = ring->times;
  P.feats = static_cast<uint8_t*>(ring->feats);
  P.wp = ring->write_pos;
  P.eids = ring->eids;
  P.nbase = P.lst;
  P.status = status;

  vec = 2;
  if (P.row_bytes % 16 == 0 && aligned16(ring->feats) && (feat == nullptr || aligned16(feat)))
    vec = 16;
  else if (P.row_bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(ring->feats) & 3u) == 0 &&
           (feat == nullptr || (reinterpret_cast<uintptr_t>(feat) & 3u) == 0))
    vec = 4;
  const int64_t nchunks = P.row_bytes / vec;
  int tpe_log2 = 0;
  // lanes per singleton entry: one chunk each up to 16 lanes, then several per lane
  while ((int64_t(1) << tpe_log2) < nchunks && tpe_log2 < 4) ++tpe_log2;
  P.tpe_log2 = tpe_log2;
  const int64_t epb = kThreads >> tpe_log2;
  P.ga = static_cast<int>((n + epb - 1) / epb);
  // small / large group roles loop over the device-side group counts, so their
  // block counts are capped instead of sized for the worst case (n/2, n/65 groups)
  P.gb = static_cast<int>(std::min<int64_t>((n / 2 + kCommitWaves) / kCommitWaves, kSmallGroupBlocks));
  return TGX_OK;
}

template <int VEC>
void launch_commit_vec(const AppendParams& P, hipStream_t stream) {
  if (plan_fused_ok(P)) {
    const int64_t epb = kKeptThreads >> P.tpe_log2;
    hipLaunchKernelGGL(kept_commit<VEC>, dim3(static_cast<unsigned>((P.n + epb - 1) / epb)),
                       dim3(kKeptThreads), 0, stream, P);
  } else {
    const int64_t gc = std::min<int64_t>(P.n / (kWave + 1) + 1, kLargeGroupBlocks);
    hipLaunchKernelGGL(append_commit<VEC>, dim3(static_cast<unsigned>(P.ga + P.gb + gc)),
                       dim3(kThreads), 0, stream, P);
  }
}

int launch_commit(const AppendParams& P, int vec, hipStream_t stream) {
  switch (vec) {
    case 16:
      launch_commit_vec<16>(P, stream);
      break;
    case 4:
      launch_commit_vec<4>(P, stream);
      break;
    default:
      launch_commit_vec<2>(P, stream);
      break;
  }
  return check_launch(plan_fused_ok(P) ? "kept_commit" : "append_commit");
}

}  // namespace
}  // namespace tgx

extern "C" int tgx_ring_append(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                               const double* time, const void* feat, int64_t b,
                               int64_t eid_base, void* workspace, size_t workspace_bytes,
                               int32_t* status, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  AppendParams P;
  int vec;
  int rc = setup_append("tgx_ring_append", ring, src, dst, time, feat, b, eid_base, workspace,
                        workspace_bytes, status, P, vec);
  if (rc != TGX_OK || b == 0) return rc;
  if ((rc = launch_plan(P, stream))) return rc;
  return launch_commit(P, vec, stream);
}

extern "C" int tgx_ring_plan(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                             const double* time, int64_t b, void* workspace, size_t workspace_bytes,
                             void* stream_) {
  PlanParams P;
  int rc = plan_setup("tgx_ring_plan", ring, src, dst, time, b, workspace, workspace_bytes, P);
  if (rc != TGX_OK || b == 0) return rc;
  return launch_plan(P, static_cast<hipStream_t>(stream_));
}

extern "C" int tgx_ring_commit(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                               const double* time, const void* feat, int64_t b, int64_t eid_base,
                               void* workspace, size_t workspace_bytes, int32_t* status,
                               void* stream_) {
  AppendParams P;
  int vec;
  int rc = setup_append("tgx_ring_commit", ring, src, dst, time, feat, b, eid_base, workspace,
                        workspace_bytes, status, P, vec);
  if (rc != TGX_OK || b == 0) return rc;
  return launch_commit(P, vec, static_cast<hipStream_t>(stream_));
}

extern "C" int tgx_ring_discard(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                                int64_t b, void* workspace, size_t workspace_bytes, void* stream_) {
  // the plan's time array is not read by the discard
  static const double kNoTime = 0.0;
  PlanParams P;
  int rc = plan_setup("tgx_ring_discard", ring, src, dst, &kNoTime, b, workspace, workspace_bytes, P);
  if (rc != TGX_OK || b == 0) return rc;
  const dim3 grid1(static_cast<unsigned>((P.n + kThreads - 1) / kThreads));
  hipLaunchKernelGGL(append_discard, grid1, dim3(kThreads), 0, static_cast<hipStream_t>(stream_), P,
                     plan_fused_ok(P) ? 1 : 0);
  return check_launch("append_discard");
}

// ---- tgx_ring_append_static: the workspace in a file-scope device array ----
namespace tgx {
namespace {

constexpr size_t kStaticWorkspaceBytes = size_t(2) << 20;  // 2 MiB per GPU
constexpr int kMaxDevices = 64;

// The static workspace.  Its name is a host-side stand-in: kernels get the
// device address that hipGetSymbolAddress returns for the current device.
__device__ __align__(256) uint8_t scratch[kStaticWorkspaceBytes];

std::mutex g_static_mu;
void* g_static_ptr[kMaxDevices] = {};

// device address of `scratch` on the current device, resolved once per device
int static_workspace(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TGX_ERR_HIP, "tgx_ring_append_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TGX_ERR_LIMIT, "tgx_ring_append_static: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (g_static_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(TGX_ERR_HIP, "tgx_ring_append_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_static_ptr[dev] = p;
  }
  *out = g_static_ptr[dev];
  return TGX_OK;
}

}  // namespace
}  // namespace tgx

extern "C" size_t tgx_ring_append_static_max_bytes(void) { return kStaticWorkspaceBytes; }

extern "C" int tgx_ring_append_static(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                                      const double* time, const void* feat, int64_t b,
                                      int64_t eid_base, int32_t* status, void* stream) {
  if (b < 0) return fail(TGX_ERR_ARG, "tgx_ring_append_static: negative batch size %lld", (long long)b);
  if (b == 0) return ring == nullptr ? fail(TGX_ERR_ARG, "tgx_ring_append_static: ring is NULL") : TGX_OK;
  if (b >= (int64_t(1) << 29) || tgx_ring_append_workspace_size(b) > kStaticWorkspaceBytes)
    return fail(TGX_ERR_LIMIT, "tgx_ring_append_static: %lld events need %zu workspace bytes, the "
                "static workspace holds %zu", (long long)b,
                b < (int64_t(1) << 29) ? tgx_ring_append_workspace_size(b) : size_t(0),
                kStaticWorkspaceBytes);
  void* ws = nullptr;
  const int rc = static_workspace(&ws);
  if (rc != TGX_OK) return rc;
  return tgx_ring_append(ring, src, dst, time, feat, b, eid_base, ws, kStaticWorkspaceBytes, status,
                         stream);
}
