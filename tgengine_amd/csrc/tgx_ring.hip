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
// Design: four launches on the caller's stream, all spread over the device.
//   1. count  : per-node tickets from node-indexed counters owned by the ring
//               (zero between calls); equal nodes inside a wavefront are
//               matched first so a hot node costs one atomic per wavefront.
//   2. groups : the ticket-0 entry of every node seen more than once reserves
//               a contiguous list of c slots and a group id, small (c <= 64)
//               or large (one atomic per wave, offsets by a wave scan).
//   3. fill   : list[base[u] + ticket] = entry index.
//   4. commit : singletons (c == 1) are written directly; a small group is
//               ranked by one wavefront in registers, a large group by a whole
//               workgroup over LDS bitmaps of 8192-index windows walked down
//               from the top of the batch; kept entries are written, count[u]
//               is restored to zero and write_pos advances.
// Feature rows move as 16-byte vectors when the row allows it.
#include "tgx_internal.h"

namespace tgx {
namespace {

constexpr int kThreads = 256;
constexpr int kCommitWaves = kThreads / kWave;
constexpr int kWinBits = 8192;                 // bitmap window (indices)
constexpr int kWinWords = kWinBits / 32;       // 256 words = 1 KB
static_assert(kWinWords == kThreads, "one bitmap word per thread");
enum { kCtlCursor = 0, kCtlGroups = 1, kCtlTimeOk = 2, kCtlLarge = 3 };

// (write_pos + off) % B for write_pos >= 0, 0 <= off < B
__device__ __forceinline__ int64_t ring_slot(int64_t w, int off, int B) {
  const uint64_t x = static_cast<uint64_t>(w) + static_cast<uint64_t>(off);
  if ((B & (B - 1)) == 0) return static_cast<int64_t>(x & static_cast<uint64_t>(B - 1));
  if (x < (uint64_t(1) << 32))
    return static_cast<int64_t>(static_cast<uint32_t>(x) % static_cast<uint32_t>(B));
  return static_cast<int64_t>(x % static_cast<uint64_t>(B));
}

__device__ __forceinline__ int64_t entry_node(const int64_t* src, const int64_t* dst, int64_t i,
                                              int64_t b) {
  return i < b ? src[i] : dst[i - b];
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

struct AppendParams {
  const int64_t* src;
  const int64_t* dst;
  const double* time;
  const uint8_t* feat;  // [b, row_bytes] or null (zero rows)
  int64_t b;
  int64_t n;
  int64_t N;
  int B;
  int64_t row_bytes;
  int64_t eid_base;
  int32_t* ids;
  double* times;
  uint8_t* feats;
  int64_t* wp;
  int64_t* eids;
  int32_t* cnt;     // [N] per-node counters (zero between calls)
  int32_t* nbase;   // [N] list base of multi-entry nodes
  int32_t* ctl;     // [16] cursor, group count, time flag
  int32_t* ticket;  // [n]
  int32_t* list;    // [n]
  int32_t* groups;  // [n/2 + 1] small groups
  int32_t* large;   // [n/65 + 1] large groups
  int32_t* status;
  int tpe_log2;     // lanes per entry (singleton copy)
  int ga;           // blocks of the singleton role in commit
  int gb;           // blocks of the small-group role
};

// ---- 1. count -------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void append_count(AppendParams P) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  if (i == 0) {
    P.ctl[kCtlCursor] = 0;
    P.ctl[kCtlGroups] = 0;
    P.ctl[kCtlLarge] = 0;
  }
  int bad = 0;
  bool time_ok = false;
  int32_t u = -1;
  if (i < P.n) {
    const int64_t uu = entry_node(P.src, P.dst, i, P.b);
    if (uu < 0 || uu >= P.N)
      bad = 1;
    else
      u = static_cast<int32_t>(uu);
    // reference key from*(int(max t)+2)+i is lexicographic iff int(max t)+2 > n-1
    if (i < P.b) time_ok = trunc(P.time[i]) > static_cast<double>(P.n - 3);
  }
  // match equal nodes inside the wavefront: one atomic per distinct node
  const uint64_t active = __ballot(u >= 0);
  uint64_t todo = active;
  uint64_t peers = 0;
  while (todo) {
    const int j = __ffsll(static_cast<unsigned long long>(todo)) - 1;
    const int32_t uj = __shfl(u, j, kWave);
    const uint64_t m = __ballot(u == uj) & active;
    if ((m >> lane) & 1) peers = m;
    todo &= ~m;
  }
  if (u >= 0) {
    const int leader = __ffsll(static_cast<unsigned long long>(peers)) - 1;
    const int rank = __popcll(peers & ((uint64_t(1) << lane) - 1));
    int base = 0;
    if (lane == leader) base = atomicAdd(&P.cnt[u], __popcll(peers));
    // leader lanes publish their base; every lane reads its leader's
    base = __shfl(base, leader, kWave);
    P.ticket[i] = base + rank;
  } else if (i < P.n) {
    P.ticket[i] = -1;
  }
  const uint64_t bm = __ballot(bad);
  const uint64_t tm = __ballot(time_ok);
  if (lane == 0) {
    if (bm && P.status != nullptr) atomicAdd(&P.status[TGX_ST_BAD_EVENT_NODE], __popcll(bm));
    if (tm) atomicOr(&P.ctl[kCtlTimeOk], 1);
  }
}

// ---- 2. groups --------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void append_groups(AppendParams P) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  if (i == 0) {
    if (P.ctl[kCtlTimeOk] == 0 && P.status != nullptr)
      atomicAdd(&P.status[TGX_ST_KEY_COLLISION], 1);
    P.ctl[kCtlTimeOk] = 0;
  }
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

// ---- 3. fill ----------------------------------------------------------------
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

// copy the kept rows R[0..kept) of node u (row r -> slot (w + kept - 1 - r) % B);
// threads t = first, first + stride, ... of the caller share the work
template <int VEC>
__device__ __forceinline__ void write_kept(const AppendParams& P, const int32_t* R, int64_t u,
                                           int kept, int64_t w, int first, int stride) {
  using V = typename VecT<VEC>::T;
  const int nv = static_cast<int>(P.row_bytes / VEC);
  for (int r = first; r < kept; r += stride)
    write_entry_meta(P, R[r], u * P.B + ring_slot(w, kept - 1 - r, P.B));
  const int total = kept * nv;
  for (int f = first; f < total; f += stride) {
    const int r = f / nv;
    const int cch = f - r * nv;
    const int64_t i = R[r];
    const int64_t e = i < P.b ? i : i - P.b;
    const int64_t slot = u * P.B + ring_slot(w, kept - 1 - r, P.B);
    V* drow = reinterpret_cast<V*>(P.feats + slot * P.row_bytes);
    drow[cch] = P.feat != nullptr ? reinterpret_cast<const V*>(P.feat + e * P.row_bytes)[cch] : V{};
  }
}

// ---- 4. commit --------------------------------------------------------------
// blocks [0, ga): singletons; [ga, ga+gb): small groups, one per wavefront;
// [ga+gb, ...): large groups, one per workgroup
template <int VEC>
__global__ __launch_bounds__(kThreads) void append_commit(AppendParams P) {
  using V = typename VecT<VEC>::T;
  __shared__ uint32_t bitmap[kWinWords];
  __shared__ int32_t sfx[kWinWords];                     // set bits in later words
  __shared__ int32_t rows[kCommitWaves][TGX_MAX_SLOTS];  // kept entry index by e
  __shared__ int32_t wsum[kCommitWaves];
  const int nv = static_cast<int>(P.row_bytes / VEC);
  const int blk = static_cast<int>(blockIdx.x);

  if (blk < P.ga) {
    // singletons: tpe lanes per entry
    const int tpe = 1 << P.tpe_log2;
    const int epb = kThreads >> P.tpe_log2;
    const int64_t i = static_cast<int64_t>(blk) * epb + (threadIdx.x >> P.tpe_log2);
    const int l = threadIdx.x & (tpe - 1);
    if (i >= P.n) return;
    if (P.ticket[i] != 0) return;
    const int64_t u = entry_node(P.src, P.dst, i, P.b);
    if (P.cnt[u] != 1) return;
    const int64_t w = P.wp[u];
    const int64_t slot = u * P.B + ring_slot(w, 0, P.B);
    const int64_t e = i < P.b ? i : i - P.b;
    V* drow = reinterpret_cast<V*>(P.feats + slot * P.row_bytes);
    if (P.feat != nullptr) {
      const V* srow = reinterpret_cast<const V*>(P.feat + e * P.row_bytes);
      for (int c = l; c < nv; c += tpe) drow[c] = srow[c];
    } else {
      for (int c = l; c < nv; c += tpe) drow[c] = V{};
    }
    if (l == 0) {
      write_entry_meta(P, i, slot);
      P.wp[u] = w + 1;
      P.cnt[u] = 0;
    }
    return;
  }

  const int wv = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (blk < P.ga + P.gb) {
    // small group (2 <= c <= 64): ranks by comparing list entries in registers
    const int64_t gid = static_cast<int64_t>(blk - P.ga) * kCommitWaves + wv;
    if (gid >= P.ctl[kCtlGroups]) return;  // wave-uniform
    const int64_t u = P.groups[gid];
    const int c = P.cnt[u];
    const int base = P.nbase[u];
    const int kept = c < P.B ? c : P.B;
    int32_t* R = rows[wv];
    const int32_t idx = lane < c ? P.list[base + lane] : -1;
    int e = 0;
    for (int j = 0; j < c; ++j) e += __shfl(idx, j, kWave) > idx;
    if (lane < c && e < kept) R[e] = idx;
    wave_sync_lds();
    const int64_t w = P.wp[u];
    write_kept<VEC>(P, R, u, kept, w, lane, kWave);
    if (lane == 0) {
      P.wp[u] = w + kept;
      P.cnt[u] = 0;
    }
    return;
  }

  // large group (c > 64): the workgroup ranks the list over bitmap windows of
  // kWinBits entry indices, from the top of the batch down, until `kept`
  // entries are found
  const int64_t gid = blk - P.ga - P.gb;
  if (gid >= P.ctl[kCtlLarge]) return;  // workgroup-uniform
  const int t = threadIdx.x;
  const int64_t u = P.large[gid];
  const int c = P.cnt[u];
  const int base = P.nbase[u];
  const int kept = c < P.B ? c : P.B;
  int32_t* R = rows[0];
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
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" size_t tgx_ring_append_workspace_size(int64_t b) {
  if (b <= 0) return 256;
  const size_t n = static_cast<size_t>(2 * b);
  return 2 * align256(n * 4) + align256((n / 2 + 1) * 4) + align256((n / 65 + 1) * 4);
}

extern "C" size_t tgx_ring_scratch_size(int64_t num_nodes) {
  if (num_nodes < 0) return 0;
  return static_cast<size_t>(2 * num_nodes + 16) * sizeof(int32_t);
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
      ring->scratch == nullptr || (ring->feats == nullptr && ring->feat_dim > 0))
    return fail(TGX_ERR_ARG,
                "tgx_ring_append: ring arrays (ids, times, feats, write_pos, scratch) must not be NULL");
  const int esz = feat_elem_bytes(ring->feat_dtype);
  if (esz == 0) return fail(TGX_ERR_DTYPE, "tgx_ring_append: unsupported feat dtype %d", ring->feat_dtype);
  if (ring->num_nodes <= 0 || ring->num_nodes >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "tgx_ring_append: num_nodes %lld outside [1, 2^31)",
                (long long)ring->num_nodes);
  if (ring->slots < 1 || ring->slots > TGX_MAX_SLOTS)
    return fail(TGX_ERR_LIMIT, "tgx_ring_append: slots %d outside [1, %d]", ring->slots,
                TGX_MAX_SLOTS);
  if (ring->feat_dim < 0) return fail(TGX_ERR_ARG, "tgx_ring_append: negative feat_dim");
  const int64_t n = 2 * b;
  if (n >= (int64_t(1) << 30)) return fail(TGX_ERR_LIMIT, "tgx_ring_append: batch too large");
  const size_t need = tgx_ring_append_workspace_size(b);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(TGX_ERR_ARG, "tgx_ring_append: workspace of %zu bytes needed, got %zu", need,
                workspace_bytes);

  AppendParams P{};
  P.src = src;
  P.dst = dst;
  P.time = time;
  P.feat = static_cast<const uint8_t*>(feat);
  P.b = b;
  P.n = n;
  P.N = ring->num_nodes;
  P.B = ring->slots;
  P.row_bytes = static_cast<int64_t>(ring->feat_dim) * esz;
  P.eid_base = eid_base;
  P.ids = ring->ids;
  P.times = ring->times;
  P.feats = static_cast<uint8_t*>(ring->feats);
  P.wp = ring->write_pos;
  P.eids = ring->eids;
  P.cnt = ring->scratch;
  P.nbase = ring->scratch + ring->num_nodes;
  P.ctl = ring->scratch + 2 * ring->num_nodes;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  P.ticket = reinterpret_cast<int32_t*>(ws);
  P.list = reinterpret_cast<int32_t*>(ws + align256(static_cast<size_t>(n) * 4));
  P.groups = reinterpret_cast<int32_t*>(ws + 2 * align256(static_cast<size_t>(n) * 4));
  P.large = reinterpret_cast<int32_t*>(ws + 2 * align256(static_cast<size_t>(n) * 4) +
                                       align256(static_cast<size_t>(n / 2 + 1) * 4));
  P.status = status;

  int vec = 2;
  if (P.row_bytes % 16 == 0 && aligned16(ring->feats) && (feat == nullptr || aligned16(feat)))
    vec = 16;
  else if (P.row_bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(ring->feats) & 3u) == 0 &&
           (feat == nullptr || (reinterpret_cast<uintptr_t>(feat) & 3u) == 0))
    vec = 4;
  const int64_t nchunks = P.row_bytes / vec;
  int tpe_log2 = 0;
  while ((int64_t(1) << tpe_log2) < nchunks && tpe_log2 < 6) ++tpe_log2;
  P.tpe_log2 = tpe_log2;
  const int64_t epb = kThreads >> tpe_log2;
  P.ga = static_cast<int>((n + epb - 1) / epb);
  P.gb = static_cast<int>((n / 2 + kCommitWaves) / kCommitWaves);  // at most n/2 groups
  const int64_t gc = n / (kWave + 1) + 1;                              // at most n/65 large
  const dim3 grid1(static_cast<unsigned>((n + kThreads - 1) / kThreads));
  const dim3 grid4(static_cast<unsigned>(P.ga + P.gb + gc));

  hipLaunchKernelGGL(append_count, grid1, dim3(kThreads), 0, stream, P);
  int rc = check_launch("append_count");
  if (rc) return rc;
  hipLaunchKernelGGL(append_groups, grid1, dim3(kThreads), 0, stream, P);
  if ((rc = check_launch("append_groups"))) return rc;
  hipLaunchKernelGGL(append_fill, grid1, dim3(kThreads), 0, stream, P);
  if ((rc = check_launch("append_fill"))) return rc;
  switch (vec) {
    case 16:
      hipLaunchKernelGGL(append_commit<16>, grid4, dim3(kThreads), 0, stream, P);
      break;
    case 4:
      hipLaunchKernelGGL(append_commit<4>, grid4, dim3(kThreads), 0, stream, P);
      break;
    default:
      hipLaunchKernelGGL(append_commit<2>, grid4, dim3(kThreads), 0, stream, P);
      break;
  }
  return check_launch("append_commit");
}
