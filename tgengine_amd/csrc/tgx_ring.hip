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
// Both designs below take per-node tickets from node-indexed counters owned by
// the ring (zero between calls); equal nodes of a workgroup are first
// aggregated in an LDS hash table, so a node costs one global atomic per
// workgroup however hot it is.  Tickets number a node's entries in no
// particular order; ranking by entry index happens when the node is written.
//
// Batches of up to kFastMaxEntries entries: two launches.
//   plan   : tickets; ticket t < kListCap stores the entry in the node's list
//            lst[u][t] (ring scratch); the ticket-1 entry appends the node to
//            the group list, the ticket-kListCap entry to the large-group
//            list.  The two cursors share one 64-bit word: one atomic per
//            workgroup.
//   commit : singletons (c == 1) are written directly; a group of
//            c <= kListCap is ranked by one wavefront from its node list; a
//            larger group by a workgroup that reads the plan's int32 node of
//            every entry from the top of the batch down, kTopChunk entries at a
//            time, and ranks the node's entries until the kept ones are found.  Every role
//            starts its loads before it knows whether it has work, so a role
//            costs two or three memory round trips.  The first small-group workgroup reports the
//            diagnostics and clears the other cursor set for the next plan
//            (two sets alternate).
// Larger batches: four launches, whose lists are sized after counting.
//   count  : tickets.
//   groups : the ticket-0 entry of every node seen more than once reserves
//            a contiguous list of c slots and a group id, small (c <= 64)
//            or large (one atomic per wave, offsets by a wave scan).
//   fill   : list[base[u] + ticket] = entry index.
//   commit : singletons as above; a small group is ranked by one wavefront in
//            registers, a large group by a whole workgroup over bitmap
//            windows walked down from the top of the batch.
// Every path writes the kept entries, restores count[u] to zero and advances
// write_pos.  Feature rows move as 16-byte vectors when the row allows it.
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
// the two-launch commit runs 512-thread workgroups, so that the large-group
// role's step of kTopChunk entries is kTopRows 16-byte loads per thread
constexpr int kFastThreads = 512;
constexpr int kFastWaves = kFastThreads / kWave;
constexpr int kTopRows = 4;                 // 16-byte loads (4 entry nodes each) in flight per thread
constexpr int kTopChunk = 4 * kTopRows * kFastThreads;  // entries per top-down step
constexpr int64_t kFastLargeBlocks = 128;   // two-launch commit blocks for large groups
constexpr int64_t kFastSmallBlocks = 128;   // two-launch commit blocks for small groups (8 waves each)

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
  int tpe_log2;     // lanes per entry (singleton copy)
  int ga;           // blocks of the singleton role in commit
  int gb;           // blocks of the small-group role
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
__global__ __launch_bounds__(kThreads) void fast_plan(PlanParams P) {
  __shared__ PlanLds L;
  plan_block(P, blockIdx.x, L);
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

// copy the kept rows R[0..kept) (kept <= kListCap) of node u (row r -> slot
// (w + kept - 1 - r) % B) by one wavefront: lanes 8r .. 8r + 7 take row r, lane
// 8r + j its chunks j, j + 8, ..., kSmallDepth of them per round, so a row of up
// to 8 kSmallDepth chunks costs one round trip
constexpr int kSmallDepth = 8;
static_assert(kListCap * 8 == kWave, "eight lanes per listed row");
template <int VEC>
__device__ __forceinline__ void write_listed(const AppendParams& P, const int32_t* R, int64_t u,
                                             int kept, int64_t w) {
  using V = typename VecT<VEC>::T;
  const int lane = threadIdx.x & (kWave - 1);
  const int r = lane >> 3;
  const int j = lane & 7;
  if (r >= kept) return;
  const int nv = static_cast<int>(P.row_bytes / VEC);
  const int64_t i = R[r];
  const int64_t e = i < P.b ? i : i - P.b;
  const int64_t slot = u * P.B + ring_slot(w, kept - 1 - r, P.B);
  const V* srow = reinterpret_cast<const V*>(P.feat + e * P.row_bytes);
  V* drow = reinterpret_cast<V*>(P.feats + slot * P.row_bytes);
  int32_t id = 0;
  double tm = 0.0;
  if (j == 0) {
    id = static_cast<int32_t>(i < P.b ? P.dst[e] : P.src[e]);
    tm = P.time[e];
  }
  for (int c0 = j; c0 < nv || j == 0; c0 += 8 * kSmallDepth) {
    V v[kSmallDepth];
#pragma unroll
    for (int k = 0; k < kSmallDepth; ++k) {
      const int c = c0 + 8 * k;
      v[k] = (P.feat != nullptr && c < nv) ? srow[c] : V{};
    }
    if (j == 0 && c0 == 0) {
      P.ids[slot] = id;
      P.times[slot] = tm;
      if (P.eids != nullptr) P.eids[slot] = P.eid_base + e;
    }
#pragma unroll
    for (int k = 0; k < kSmallDepth; ++k) {
      const int c = c0 + 8 * k;
      if (c < nv) drow[c] = v[k];
    }
    if (c0 + 8 * kSmallDepth >= nv) break;
  }
}

// one group of c <= kWave entries listed in idx (lane j < c holds one entry
// index), ranked in registers by one wavefront, then written (LISTED: c <=
// kListCap, copied by write_listed)
template <int VEC, bool LISTED = false>
__device__ __forceinline__ void commit_small(const AppendParams& P, int64_t u, int c, int32_t idx,
                                             int64_t w, int32_t* R) {
  const int lane = threadIdx.x & (kWave - 1);
  const int kept = c < P.B ? c : P.B;
  int e = 0;
  for (int j = 0; j < c; ++j) e += __shfl(idx, j, kWave) > idx;
  if (lane < c && e < kept) R[e] = idx;
  wave_sync_lds();
  if constexpr (LISTED)
    write_listed<VEC>(P, R, u, kept, w);
  else
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
// The plan's node of every entry, four per 16-byte load, top-down: row r of
// thread t holds entries 4q .. 4q + 3 of q = hi4 / 4 - 1 - (r kFastThreads + t)
// (hi4 a multiple of 4; the node array is padded to whole 256-byte lines, and
// indices >= n are masked by the caller), so each row covers 4 kFastThreads
// consecutive entries in descending order.
__device__ __forceinline__ void load_top(const AppendParams& P, int64_t hi4,
                                         int4 (&nd)[kTopRows]) {
#pragma unroll
  for (int r = 0; r < kTopRows; ++r) {
    const int64_t q = hi4 / 4 - 1 - (static_cast<int64_t>(r) * kFastThreads + threadIdx.x);
    nd[r] = q >= 0 ? reinterpret_cast<const int4*>(P.ticket)[q] : make_int4(-1, -1, -1, -1);
  }
}

// LDS of the top-down ranking: the match count of every (row, wavefront)
struct TopLds {
  int32_t tot[kTopRows][kFastWaves];
};
static_assert(kTopRows * kFastWaves <= kWave, "one lane per (row, wavefront) count");

// set bits of the wave mask b below this lane
__device__ __forceinline__ int lanes_below(uint64_t b) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b), 0u)));
}

// One large group (c > kListCap) by the whole workgroup.  Its kept entries are
// its last kept = min(c, B) in the batch: the plan's node array is read from the
// top down, kTopChunk entries per step, and the entry with e later entries of
// node u is ranked from the match counts (matches in earlier steps, earlier
// rows, lower wavefronts, lower lanes, and this lane's higher entries).  Within
// a wavefront, three ballots of the bits of every lane's count give the
// matches of the lower lanes (mbcnt) and the wavefront's total, so only the
// (row, wavefront) totals pass through LDS.  The first step (nd) is loaded by
// the caller before u is known.  Steps end once B entries are found (kept = B)
// or the batch is exhausted (kept = c), so the node's counter is not read.
template <int VEC>
__device__ __forceinline__ void fast_large(const AppendParams& P, int64_t u, int4 (&nd)[kTopRows],
                                           int32_t* R, TopLds& T) {
  const int wv = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int t = threadIdx.x;
  const int32_t u32 = static_cast<int32_t>(u);
  const int n32 = static_cast<int>(P.n);  // < 2^30 entries, so entry indices fit in int
  int carry = 0;
  for (int hi4 = (n32 + 3) & ~3;;) {  // workgroup-uniform
    // m4[r] bit s: entry 4q + 3 - s of row r is node u (s = 0 is the highest);
    // below[r]: matches of the lower lanes of this wavefront in row r
    uint32_t m4[kTopRows];
    int below[kTopRows];
#pragma unroll
    for (int r = 0; r < kTopRows; ++r) {
      const int top = hi4 - 4 * (r * kFastThreads + t) - 1;  // 4q + 3
      uint32_t m = static_cast<uint32_t>(nd[r].w == u32) | static_cast<uint32_t>(nd[r].z == u32) << 1 |
                   static_cast<uint32_t>(nd[r].y == u32) << 2 | static_cast<uint32_t>(nd[r].x == u32) << 3;
      // entries n .. hi4 - 1 (at most 3, in the topmost load of the first step)
      // hold stale nodes: entry top - s is valid iff s >= top - n + 1
      if (top >= n32) m &= (0xfu << (top - n32 + 1)) & 0xfu;
      m4[r] = m;
      const int cnt = __popc(m);
      int bl = 0, tot = 0;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const uint64_t b = __ballot((cnt >> k) & 1);
        bl += lanes_below(b) << k;
        tot += __popcll(b) << k;
      }
      below[r] = bl;
      if (lane == 0) T.tot[r][wv] = tot;
    }
    __syncthreads();
    // lane l < kTopRows kFastWaves: the count of (row l / kFastWaves,
    // wavefront l % kFastWaves); an exclusive scan in that order gives bases
    const int x = lane < kTopRows * kFastWaves ? T.tot[lane / kFastWaves][lane % kFastWaves] : 0;
    // inclusive scan over lanes [0, 32) in registers (DPP): shifts by 1, 2, 4
    // and 8 lanes within each 16-lane row, then row 0's last lane into row 1
    static_assert(kTopRows * kFastWaves == 32, "the scan covers two DPP rows");
    int incl = x;
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xf, 0xf, false);  // row_shr:1
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xf, 0xf, false);  // row_shr:2
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xf, 0xf, false);  // row_shr:4
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xf, 0xf, false);  // row_shr:8
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1, 3
    // the lane index is wavefront-uniform: read the bases with readlane
    const int step_total = __builtin_amdgcn_readlane(incl, kTopRows * kFastWaves - 1);
    const int exc = incl - x;
    const int wvu = __builtin_amdgcn_readfirstlane(wv);
#pragma unroll
    for (int r = 0; r < kTopRows; ++r) {
      int e = carry + __builtin_amdgcn_readlane(exc, r * kFastWaves + wvu) + below[r];
      uint32_t m = m4[r];
      const int top = hi4 - 4 * (r * kFastThreads + t) - 1;
      // only ranks below B are kept
      for (; m != 0u && e < P.B; m &= m - 1, ++e) R[e] = top - __builtin_ctz(m);
    }
    carry += step_total;
    hi4 -= kTopChunk;
    __syncthreads();  // T is rewritten by the next step; R is complete at the end
    if (carry >= P.B || hi4 <= 0) break;
    load_top(P, hi4, nd);
  }
  const int kept = carry < P.B ? carry : P.B;
  // the write position is loaded here, not with the node: the step loop's
  // first wait would otherwise wait for it too (one round trip more); here it
  // shares the round trip of the kept rows' loads
  const int64_t w = P.wp[u];
  write_kept<VEC>(P, R, u, kept, w, t, kFastThreads);
  if (t == 0) {
    P.wp[u] = w + kept;
    P.cnt[u] = 0;
  }
  __syncthreads();  // the next group rewrites R
}

// the plan's cursor word (groups | large counts) of ctl words 8-15 (c0, c1:
// both cursor sets, phase_next, phase_cur)
static_assert(kCtlPhaseCur - kCtlFCursor - 4 == 1, "phase_cur is word 1 of c1");
__device__ __forceinline__ uint64_t plan_cursor(u32x4 c0, u32x4 c1) {
  const uint32_t ph = c1.y & 1u;
  return ph == 0 ? (static_cast<uint64_t>(c0.y) << 32 | c0.x) : (static_cast<uint64_t>(c0.w) << 32 | c0.z);
}

// the first small-group workgroup of a commit (gb >= 1 always), once the
// cursor words are in: report the plan's diagnostics, clear them, clear the
// other cursor set (its plan is committed) and hand it to the next plan
__device__ __forceinline__ void fast_diagnostics(const AppendParams& P, uint32_t phase_cur) {
  const int ph = static_cast<int>(phase_cur & 1u);
  const u32x4 dg = *reinterpret_cast<const u32x4*>(P.ctl + kCtlFDiag);
  const int time_flag = static_cast<int>(ph == 0 ? dg[0] : dg[2]);
  const int bad = static_cast<int>(ph == 0 ? dg[1] : dg[3]);
  *reinterpret_cast<uint64_t*>(P.ctl + kCtlFCursor + 2 * (1 - ph)) = 0;
  P.ctl[kCtlPhaseNext] = 1 - ph;
  if (P.status != nullptr) {
    if (bad != 0) atomicAdd(&P.status[TGX_ST_BAD_EVENT_NODE], bad);
    if (time_flag == 0) atomicAdd(&P.status[TGX_ST_KEY_COLLISION], 1);
  }
  P.ctl[kCtlFDiag + 2 * ph] = 0;
  P.ctl[kCtlFDiag + 2 * ph + 1] = 0;
}

// blocks [0, ga): singletons; [ga, ga+gb): groups of c <= kListCap, one per
// wavefront; [ga+gb, ...): larger groups, one per workgroup.  The ctl words
// (cursors, phase) are loaded first, and every role issues its own first loads
// before it uses them, so they cost one round trip together: loads and their
// wait counter are in order, and a wait for a younger load is a wait for all.
template <int VEC>
__global__ __launch_bounds__(kFastThreads) void fast_commit(AppendParams P) {
  __shared__ int32_t rows[kFastWaves][TGX_MAX_SLOTS];
  __shared__ TopLds top;
  const int blk = static_cast<int>(blockIdx.x);
  const int wv = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  // ctl words 8-15 in one round trip: both cursor sets, phase_next, phase_cur
  // (this launch writes only the other set and phase_next, which it does not use)
  const u32x4 c0 = *reinterpret_cast<const u32x4*>(P.ctl + kCtlFCursor);
  const u32x4 c1 = *reinterpret_cast<const u32x4*>(P.ctl + kCtlFCursor + 4);
  if (blk < P.ga) {
    commit_singletons<VEC>(P, blk);
  } else if (blk < P.ga + P.gb) {
    // the first group id of this wavefront is read with the cursor (in bounds of
    // the n/2 + 1 list), so a group costs three round trips
    const int gstride = P.gb * kFastWaves;
    int gid = (blk - P.ga) * kFastWaves + wv;
    int64_t u = gid <= P.n / 2 ? P.groups[gid] : 0;
    const int ngroups = field(plan_cursor(c0, c1), kFGroups);
    if (blk == P.ga && threadIdx.x == 0) fast_diagnostics(P, c1.y);
    for (; gid < ngroups; gid += gstride) {  // wave-uniform
      const int c = P.cnt[u];
      const int64_t w = P.wp[u];
      const int32_t idx = lane < kListCap ? P.lst[u * kListCap + lane] : -1;
      const int64_t u_next = gid + gstride < ngroups ? P.groups[gid + gstride] : 0;
      // a larger group has its own role; its counter reads c > kListCap, or 0
      // once that role restored it
      if (c >= 2 && c <= kListCap) commit_small<VEC, true>(P, u, c, lane < c ? idx : -1, w, rows[wv]);
      u = u_next;
    }
  } else {
    // the group's node and the top of the batch are read with the cursor
    // (gid < n / (kListCap + 1) + 1, the large list's length)
    const int gstride = static_cast<int>(gridDim.x) - P.ga - P.gb;
    const int64_t hi4 = (P.n + 3) & ~int64_t(3);
    int gid = blk - P.ga - P.gb;
    int64_t u = P.large[gid];
    int4 nd[kTopRows];
    load_top(P, hi4, nd);
    const int nlarge = field(plan_cursor(c0, c1), kFLarge);
    for (; gid < nlarge; gid += gstride) {  // workgroup-uniform
      fast_large<VEC>(P, u, nd, rows[0], top);
      if (gid + gstride < nlarge) {
        u = P.large[gid + gstride];
        load_top(P, hi4, nd);
      }
    }
  }
}

// ---- discard: restore the scratch of a planned batch without committing it ----
__global__ __launch_bounds__(kThreads) void append_discard(PlanParams P, int two_launch) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i == 0) {
    if (two_launch) {
      // the replacement plan takes the same set again (phase_next is unchanged)
      const int ph = P.ctl[kCtlPhaseCur] & 1;
      *reinterpret_cast<uint64_t*>(P.ctl + kCtlFCursor + 2 * ph) = 0;
      P.ctl[kCtlFDiag + 2 * ph] = 0;
      P.ctl[kCtlFDiag + 2 * ph + 1] = 0;
    } else {
      P.ctl[kCtlTimeOk] = 0;
      P.ctl[kCtlBad] = 0;
    }
  }
  if (i >= P.n) return;
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
  // ticket | four-launch lists | groups | large
  return align256(n * 4) + align256(n * 4) + align256((n / 2 + 1) * 4) +
         align256((n / (kListCap + 1) + 1) * 4);
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
  P.large = reinterpret_cast<int32_t*>(ws + o_groups + align256(static_cast<size_t>(n / 2 + 1) * 4));
  return TGX_OK;
}

int launch_plan(const PlanParams& P, hipStream_t stream) {
  const dim3 grid1(static_cast<unsigned>((P.n + kThreads - 1) / kThreads));
  if (plan_fused_ok(P)) {
    hipLaunchKernelGGL(fast_plan, grid1, dim3(kThreads), 0, stream, P);
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
    // 512-thread workgroups: the roles' block counts for that size
    AppendParams Q = P;
    const int64_t epb = kFastThreads >> Q.tpe_log2;
    Q.ga = static_cast<int>((Q.n + epb - 1) / epb);
    Q.gb = static_cast<int>(std::min<int64_t>((Q.n / 2 + kFastWaves) / kFastWaves, kFastSmallBlocks));
    const int64_t gc = std::min<int64_t>(Q.n / (kListCap + 1) + 1, kFastLargeBlocks);
    hipLaunchKernelGGL(fast_commit<VEC>, dim3(static_cast<unsigned>(Q.ga + Q.gb + gc)),
                       dim3(kFastThreads), 0, stream, Q);
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
  return check_launch(plan_fused_ok(P) ? "fast_commit" : "append_commit");
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
