// The plan half of the ring update (kernel a), shared by the stand-alone ring
// kernels (tgx_ring.hip) and the plan role fused into the gather launch
// (tgx_recent.hip).
//
// A plan reads the batch's src/dst/time and the ring's write positions, and
// writes only the ring's scratch and the caller's workspace, never the ring
// arrays, so it can run in the same launch as a gather over the ring.
//
// Batches of up to kFastMaxEntries entries (the two-launch update): the plan
// gives every entry its rank among its node's entries in entry order, so it can
// tell the kept ones and their final slots, and the commit is one copy per
// entry.  Each plan workgroup takes blockDim consecutive entries; it learns how
// many entries of each of its nodes come before and after its range by scanning
// the batch's node ids (inputs, immutable during the launch: no workgroup
// waits for another, and nothing passes between workgroups), and ranks its own
// entries in index order by wavefront ballots.  Larger batches: tickets from
// node-indexed counters, in no particular order, ranked when the node is
// written (four launches).
#pragma once

#include "tgx_internal.h"

namespace tgx {

constexpr int kListCap = 8;                 // node-list entries per node (ring scratch)
constexpr int64_t kFastMaxEntries = 32768;  // two-launch update up to this many entries
constexpr int kPlanMaxThreads = 512;        // plan workgroups of 64..512 threads
constexpr int kPlanMaxWaves = kPlanMaxThreads / kWave;
constexpr int kPlanHashBits = 10;           // LDS hash of equal nodes, at most half full
constexpr int kPlanHash = 1 << kPlanHashBits;
static_assert(kPlanHash >= 2 * kPlanMaxThreads, "hash table at most half full");

// ctl words (ring scratch).  Four-launch: cursors and diagnostics (words 0-4).
// Two-launch: the plan's diagnostics (words 16, 17: time flag, bad count), which
// its commit reports and clears (a discard clears them).
enum {
  kCtlCursor = 0, kCtlGroups = 1, kCtlTimeOk = 2, kCtlLarge = 3, kCtlBad = 4,
  kCtlKTime = 16, kCtlKBad = 17
};
constexpr int kCtlWords = 32;

// ring scratch: counters [N] | node lists [N, kListCap] | ctl (16-byte aligned)
inline int64_t ctl_offset(int64_t num_nodes) {
  return ((1 + kListCap) * num_nodes + 3) & ~int64_t(3);
}

struct PlanParams {
  const int64_t* src;
  const int64_t* dst;
  const double* time;
  int64_t b;
  int64_t n;       // 2b entries
  int64_t N;
  int32_t* cnt;    // [N] four-launch per-node counters (zero between calls)
  int32_t* lst;    // [N, kListCap] four-launch node lists
  int32_t* ctl;    // [kCtlWords]
  int32_t* ticket; // [n] four-launch tickets
  int32_t* list;   // [n] four-launch lists
  int32_t* groups; // [n/2 + 1] four-launch groups
  int32_t* large;  // [n/(kListCap+1) + 1] four-launch large groups
  // two-launch
  const int64_t* wpos;  // ring write positions (read)
  int B;              // ring slots
  int64_t* krec;      // [n, 2] per entry: ring slot (-1: not kept), new write position (-1: none)
};

struct PlanLds {
  int32_t hkey[kPlanHash];
  int32_t hcnt[kPlanHash];
  int32_t hbase[kPlanHash];
  uint64_t wofs[kPlanMaxWaves + 1];
};

__device__ __forceinline__ int64_t entry_node(const int64_t* src, const int64_t* dst, int64_t i,
                                              int64_t b) {
  return i < b ? src[i] : dst[i - b];
}

// node of entry i (-1 when outside [0, N): counted as a bad entry) and whether
// its event time keeps the reference key from*(int(max t)+2)+i lexicographic
// (int(max t)+2 > n-1)
__device__ __forceinline__ int32_t entry_prologue(const PlanParams& P, int64_t i, int& bad,
                                                  bool& time_ok) {
  bad = 0;
  time_ok = false;
  if (i >= P.n) return -1;
  const int64_t uu = entry_node(P.src, P.dst, i, P.b);
  if (i < P.b) time_ok = trunc(P.time[i]) > static_cast<double>(P.n - 3);
  if (uu < 0 || uu >= P.N) {
    bad = 1;
    return -1;
  }
  return static_cast<int32_t>(uu);
}

// Ticket of the entry of node u (>= 0), or -1 for u < 0.  Equal nodes of the
// workgroup are aggregated in an LDS hash table (open addressing, at most half
// full): each lane takes a local rank from its node's slot, then one global
// atomic per distinct node reserves the workgroup's tickets.
__device__ __forceinline__ int32_t node_ticket(const PlanParams& P, int32_t u, PlanLds& L) {
  for (int s = threadIdx.x; s < kPlanHash; s += blockDim.x) {
    L.hkey[s] = -1;
    L.hcnt[s] = 0;
  }
  __syncthreads();
  int hs = -1, rank = 0;
  if (u >= 0) {
    hs = static_cast<int>((static_cast<uint32_t>(u) * 2654435761u) >> (32 - kPlanHashBits));
    while (true) {  // terminates: fewer keys than slots
      const int32_t old = atomicCAS(&L.hkey[hs], -1, u);
      if (old == -1 || old == u) break;
      hs = (hs + 1) & (kPlanHash - 1);
    }
    rank = atomicAdd(&L.hcnt[hs], 1);
  }
  __syncthreads();
  for (int s = threadIdx.x; s < kPlanHash; s += blockDim.x)
    if (L.hkey[s] >= 0) L.hbase[s] = atomicAdd(&P.cnt[L.hkey[s]], L.hcnt[s]);
  __syncthreads();
  return u >= 0 ? L.hbase[hs] + rank : -1;
}

// out-of-range entries and the time flag into the words time_word / bad_word
__device__ __forceinline__ void report_diagnostics(const PlanParams& P, int bad, bool time_ok,
                                                   int time_word, int bad_word) {
  const uint64_t bm = __ballot(bad);
  const uint64_t tm = __ballot(time_ok);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    if (bm) atomicAdd(&P.ctl[bad_word], __popcll(bm));
    if (tm) atomicOr(&P.ctl[time_word], 1);
  }
}

// Ordered ranking of entries [block * T, +T), T = blockDim.x (a multiple of
// kWave, at most kOrderedMaxThreads; every thread of the workgroup calls it):
// each entry's rank among its node's entries of the batch in entry order, and
// the node's count (rank_block below; the two-launch ring plan and the negative
// pool's update build on it).
//
// LDS, plan_lds_bytes(T) (sized so that a gather launch carrying the plan keeps
// its occupancy), per slot of a hash table of the workgroup's nodes (H >= 2T
// slots, so at most half full):
//   hkey[H]          the node;
//   hba[H][4]        entries of the batch before (low 16 bits) and after (high
//                    16 bits) the range that the scan met, in four counter sets
//                    (wavefront w counts into set w % 4; both sums < 2^15);
//   wcnt[H][stride]  per wavefront, the node's entries in its part of the range
//                    (bytes; stride = 4, 8 or 16 >= T / 64).
// One 16-byte read of hba and one read of wcnt give an entry everything it
// needs at the end.
//
// SCAN: node ids each thread loads per step of the batch scan (the next step's
// loads go out before this step's lookups, the first step's before anything
// else).  A wavefront's 64 scanned entries lie all before or all after the
// range (both are multiples of 64), and its matches of one node (a hub) add up
// in one atomic.
constexpr int kOrderedMaxThreads = 1024;
constexpr int kPlanSets = 4;  // counter sets of the scan
__host__ __device__ constexpr int plan_hash_bits(int T) {
  return T > 512 ? 11 : T > 256 ? 10 : T > 128 ? 9 : T > 64 ? 8 : 7;
}
__host__ __device__ constexpr int plan_wcnt_stride(int T) { return T > 512 ? 16 : T > 256 ? 8 : 4; }
__host__ __device__ constexpr size_t plan_lds_bytes(int T) {
  return static_cast<size_t>(1 << plan_hash_bits(T)) *
         static_cast<size_t>(4 + 4 * kPlanSets + plan_wcnt_stride(T));
}

__device__ __forceinline__ int plan_hash(int32_t u, int bits) {
  return static_cast<int>((static_cast<uint32_t>(u) * 2654435761u) >> (32 - bits));
}

// sum of the four bytes of x, and of those below byte `upto` (0..4)
__device__ __forceinline__ uint32_t byte_sum(uint32_t x) { return __builtin_amdgcn_sad_u8(x, 0u, 0u); }
__device__ __forceinline__ uint32_t byte_sum_below(uint32_t x, int upto) {
  return upto <= 0 ? 0u : upto >= 4 ? byte_sum(x) : byte_sum(x & ((1u << (8 * upto)) - 1u));
}

// The ranking core, shared with the negative pool's update: entries i of [0, n)
// with node entry_node(src, dst, i, b) (b = n: src only).  For each entry of
// the workgroup's range it calls fin(i, u, c, r, w): u its node (-1 when outside
// [0, N)), c the node's entries in the batch, r the entry's rank among them in
// entry order, w = nval[u] (loaded early; nval may be NULL).  Returns 1 for a
// calling thread whose entry's node is out of range.
template <int SCAN, class Fin>
__device__ __forceinline__ int rank_block(const int64_t* src, const int64_t* dst, int64_t b, int64_t n,
                                          int64_t N, const int64_t* nval, int64_t block, uint8_t* smem,
                                          Fin&& fin) {
  const int T = static_cast<int>(blockDim.x);
  const int t = threadIdx.x;
  const int wv = t / kWave;
  const int lane = t & (kWave - 1);
  const int hbits = plan_hash_bits(T);
  const int H = 1 << hbits;
  const int stride = plan_wcnt_stride(T);
  int32_t* hkey = reinterpret_cast<int32_t*>(smem);                               // [H]
  uint32_t* hba = reinterpret_cast<uint32_t*>(smem + 4 * static_cast<size_t>(H));  // [H][4]
  uint8_t* wcnt = smem + static_cast<size_t>(4 + 4 * kPlanSets) * H;              // [H][stride]
  const int set = wv % kPlanSets;
  const int64_t lo = block * T;
  const int64_t hi = lo + T < n ? lo + T : n;
  const int64_t i = lo + t;
  // the entry's node, then the first step of the batch scan (node ids of the
  // entries outside [lo, hi)), all before any of them is waited for
  const int64_t uu = i < n ? entry_node(src, dst, i, b) : -1;
  const int64_t step = static_cast<int64_t>(T) * SCAN;
  int64_t nx[SCAN];
  auto fetch = [&](int64_t j0) {
#pragma unroll
    for (int k = 0; k < SCAN; ++k) {
      const int64_t j = j0 + static_cast<int64_t>(k) * T + t;
      nx[k] = (j < n && (j < lo || j >= hi)) ? entry_node(src, dst, j, b) : -1;
    }
  };
  fetch(0);
  for (int s = t; s < H; s += T) hkey[s] = -1;
  for (int s = t; s < kPlanSets * H; s += T) hba[s] = 0u;
  for (int s = t; s < stride * H / 4; s += T) reinterpret_cast<uint32_t*>(wcnt)[s] = 0u;
  __syncthreads();
  const int bad = i < n && (uu < 0 || uu >= N) ? 1 : 0;
  const int32_t u = i < n && !bad ? static_cast<int32_t>(uu) : -1;
  // the node's value is needed last
  const int64_t w = u >= 0 && nval != nullptr ? nval[u] : 0;
  int hs = -1;
  if (u >= 0) {
    hs = plan_hash(u, hbits);
    while (true) {  // terminates: fewer keys than slots
      const int32_t old = atomicCAS(&hkey[hs], -1, u);
      if (old == -1 || old == u) break;
      hs = (hs + 1) & (H - 1);
    }
  }
  // the wavefront's count per node (its byte of the node's wcnt row, by an
  // atomic on the row's word; a wavefront's LDS operations complete in order, so
  // the read after its own atomics sees them all), then the rank in entry order
  // among the wavefront's entries of the same node, by ballots over the nodes
  // it holds more than once
  int wrank = 0;
  {
    uint32_t* wcw = reinterpret_cast<uint32_t*>(wcnt);
    const int wi = u >= 0 ? (hs * stride + wv) >> 2 : 0;
    const int sh = 8 * (wv & 3);
    if (u >= 0) atomicAdd(&wcw[wi], 1u << sh);
    const int cnt = u >= 0 ? static_cast<int>((wcw[wi] >> sh) & 0xffu) : 0;
    uint64_t todo = __ballot(cnt > 1);
    while (todo != 0u) {  // wave-uniform
      const int leader = __builtin_ctzll(todo);
      const int sl = __builtin_amdgcn_readlane(hs, leader);
      const uint64_t same = __ballot(u >= 0 && hs == sl);
      if (u >= 0 && hs == sl)
        wrank = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(same >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(same), 0u)));
      todo &= ~same;
    }
  }
  __syncthreads();
  // the batch outside [lo, hi): entries of this workgroup's nodes before and
  // after it
  for (int64_t j0 = 0; j0 < n; j0 += step) {  // workgroup-uniform
    int64_t cur[SCAN];
#pragma unroll
    for (int k = 0; k < SCAN; ++k) cur[k] = nx[k];
    if (j0 + step < n) fetch(j0 + step);
#pragma unroll
    for (int k = 0; k < SCAN; ++k) {
      int s = -1;
      if (cur[k] >= 0 && cur[k] < N) {
        const int32_t x = static_cast<int32_t>(cur[k]);
        s = plan_hash(x, hbits);
        int32_t key = hkey[s];
        while (key != x && key != -1) {
          s = (s + 1) & (H - 1);
          key = hkey[s];
        }
        if (key != x) s = -1;
      }
      const uint64_t mm = __ballot(s >= 0);
      if (mm != 0u) {  // wave-uniform
        const uint32_t inc = j0 + static_cast<int64_t>(k) * T + t < lo ? 1u : 0x10000u;  // wave-uniform
        const int ld = __builtin_ctzll(mm);
        const int ls = __builtin_amdgcn_readlane(s, ld);
        const uint64_t same = __ballot(s == ls);
        if (lane == ld) atomicAdd(&hba[static_cast<size_t>(ls) * kPlanSets + set], inc * static_cast<uint32_t>(__popcll(same)));
        else if (s >= 0 && s != ls) atomicAdd(&hba[static_cast<size_t>(s) * kPlanSets + set], inc);
      }
    }
  }
  __syncthreads();
  if (i < n) {
    int c = 0, r = 0;
    if (u >= 0) {
      const uint4 ba = *reinterpret_cast<const uint4*>(&hba[static_cast<size_t>(hs) * kPlanSets]);
      const int before = static_cast<int>((ba.x & 0xffffu) + (ba.y & 0xffffu) + (ba.z & 0xffffu) + (ba.w & 0xffffu));
      const int after = static_cast<int>((ba.x >> 16) + (ba.y >> 16) + (ba.z >> 16) + (ba.w >> 16));
      const uint8_t* row = wcnt + static_cast<size_t>(hs) * stride;
      uint32_t cw[4] = {0u, 0u, 0u, 0u};
      if (stride == 16) {
        const uint4 v = *reinterpret_cast<const uint4*>(row);
        cw[0] = v.x; cw[1] = v.y; cw[2] = v.z; cw[3] = v.w;
      } else if (stride == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(row);
        cw[0] = v.x; cw[1] = v.y;
      } else {
        cw[0] = *reinterpret_cast<const uint32_t*>(row);
      }
      int mine = 0, below = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        mine += static_cast<int>(byte_sum(cw[q]));
        below += static_cast<int>(byte_sum_below(cw[q], wv - 4 * q));
      }
      c = before + mine + after;
      r = before + below + wrank;
    }
    fin(i, u, c, r, w);
  }
  return bad;
}

// The ring plan of entries [block * T, +T), on rank_block: the entry with rank r
// among the c entries of its node u is kept iff m = r - (c - kept) >= 0, kept =
// min(c, B), and lands in slot (wp[u] + m) % B; the node's last entry carries
// wp' = wp[u] + kept.  krec[i] = (slot, wp'), -1 for none.
template <int SCAN>
__device__ __forceinline__ void plan_block_ordered(const PlanParams& P, int64_t block, uint8_t* smem) {
  const int64_t i = block * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  // the time is loaded first and used last (the reference key's check)
  const double ti = i < P.b ? P.time[i] : 0.0;
  const int bad = rank_block<SCAN>(P.src, P.dst, P.b, P.n, P.N, P.wpos, block, smem,
                                   [&](int64_t e, int32_t u, int c, int r, int64_t w) {
    int64_t slot = -1, wnew = -1;
    if (u >= 0) {
      const int kept = c < P.B ? c : P.B;
      const int m = r - (c - kept);
      if (m >= 0) {
        const uint64_t x = static_cast<uint64_t>(w) + static_cast<uint64_t>(m);
        slot = static_cast<int64_t>(x % static_cast<uint64_t>(P.B));
      }
      if (r == c - 1) wnew = w + kept;
    }
    reinterpret_cast<longlong2*>(P.krec)[e] = make_longlong2(slot, wnew);
  });
  const bool time_ok = i < P.b && trunc(ti) > static_cast<double>(P.n - 3);
  report_diagnostics(P, bad, time_ok, kCtlKTime, kCtlKBad);
}

// Host side (tgx_ring.hip).  plan_setup checks the arguments of a plan and fills
// P (b == 0: nothing to plan, P.n == 0).  plan_fused_ok: the plan is the
// two-launch one, which plan_block runs in a caller's launch.  launch_plan runs
// a plan in launches of its own.
int plan_setup(const char* who, const tgx_ring* ring, const int64_t* src, const int64_t* dst,
               const double* time, int64_t b, void* workspace, size_t workspace_bytes,
               PlanParams& P);
inline bool plan_fused_ok(const PlanParams& P) { return P.n > 0 && P.n <= kFastMaxEntries; }
int launch_plan(const PlanParams& P, hipStream_t stream);

}  // namespace tgx
