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

// Two-launch plan of entries [block * T, +T), T = blockDim.x (a multiple of
// kWave, at most kPlanMaxThreads; every thread of the workgroup calls it).
// krec[i] = (slot, wp') for entry i: the entry with rank r among the c entries
// of its node u (in entry order) is kept iff r >= c - kept, kept = min(c, B),
// and lands in slot (wp[u] + r - (c - kept)) % B; the node's last entry also
// carries wp' = wp[u] + kept.  LDS (plan_lds_bytes(T), sized so that a gather
// launch carrying the plan keeps its occupancy): a hash table of the
// workgroup's nodes (hkey, H = 512 slots up to 256 threads, else 1024: at most
// half full), per node and counter set the entries of the batch before and
// after the range that the scan met (hba: before in the low, after in the high
// 16 bits, both < 2^15; wavefront w counts into set w % 4, so a hub node does
// not serialise one counter), and per node and wavefront its entries in the
// wavefront's part of the range (wcnt).
constexpr int kPlanScan = 4;  // node ids each thread loads per step of the batch scan
constexpr int kPlanSets = 4;  // counter sets of the scan
__host__ __device__ constexpr int plan_hash_bits(int T) { return T > 256 ? 10 : 9; }
__host__ __device__ constexpr size_t plan_lds_bytes(int T) {
  return static_cast<size_t>(1 << plan_hash_bits(T)) *
         (4 + 4 * static_cast<size_t>(T / kWave < kPlanSets ? T / kWave : kPlanSets) +
          static_cast<size_t>(T / kWave));
}

__device__ __forceinline__ int plan_hash(int32_t u, int bits) {
  return static_cast<int>((static_cast<uint32_t>(u) * 2654435761u) >> (32 - bits));
}

__device__ __forceinline__ void plan_block_ordered(const PlanParams& P, int64_t block, uint8_t* smem) {
  const int T = static_cast<int>(blockDim.x);
  const int t = threadIdx.x;
  const int wv = t / kWave;
  const int lane = t & (kWave - 1);
  const int nw = T / kWave;
  const int hbits = plan_hash_bits(T);
  const int H = 1 << hbits;
  const int nsets = nw < kPlanSets ? nw : kPlanSets;
  int32_t* hkey = reinterpret_cast<int32_t*>(smem);                 // [H]
  uint32_t* hba = reinterpret_cast<uint32_t*>(smem + 4 * H);         // [nsets][H]
  uint8_t* wcnt = smem + 4 * H + 4 * static_cast<size_t>(nsets) * H;  // [nw][H]
  uint32_t* mine_ba = hba + static_cast<size_t>(wv % kPlanSets) * H;
  const int64_t lo = block * T;
  const int64_t hi = lo + T < P.n ? lo + T : P.n;
  const int64_t i = lo + t;
  int bad;
  bool time_ok;
  const int32_t u = entry_prologue(P, i, bad, time_ok);
  // the write position is needed last: its load goes out first
  const int64_t w = u >= 0 ? P.wpos[u] : 0;
  for (int s = t; s < H; s += T) hkey[s] = -1;
  for (int s = t; s < nsets * H; s += T) hba[s] = 0u;
  for (int s = t; s < nw * H / 4; s += T) reinterpret_cast<uint32_t*>(wcnt)[s] = 0u;
  __syncthreads();
  int hs = -1;
  if (u >= 0) {
    hs = plan_hash(u, hbits);
    while (true) {  // terminates: fewer keys than slots
      const int32_t old = atomicCAS(&hkey[hs], -1, u);
      if (old == -1 || old == u) break;
      hs = (hs + 1) & (H - 1);
    }
  }
  // rank in the wavefront (entry order) and the wavefront's count per node
  int wrank = 0;
  {
    uint64_t todo = __ballot(u >= 0);
    while (todo != 0u) {  // wave-uniform
      const int leader = __builtin_ctzll(todo);
      const int sl = __shfl(hs, leader);
      const uint64_t same = __ballot(u >= 0 && hs == sl);
      if (u >= 0 && hs == sl)
        wrank = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(same >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(same), 0u)));
      if (lane == leader) wcnt[static_cast<size_t>(wv) * H + sl] = static_cast<uint8_t>(__popcll(same));
      todo &= ~same;
    }
  }
  __syncthreads();
  // the batch outside [lo, hi): entries of this workgroup's nodes before and
  // after it, counted per wavefront (hub nodes would serialise one counter);
  // each step's node ids are loaded one step ahead
  const int64_t step = static_cast<int64_t>(T) * kPlanScan;
  int64_t nx[kPlanScan];
  auto fetch = [&](int64_t j0) {
#pragma unroll
    for (int k = 0; k < kPlanScan; ++k) {
      const int64_t j = j0 + static_cast<int64_t>(k) * T + t;
      nx[k] = (j < P.n && (j < lo || j >= hi)) ? entry_node(P.src, P.dst, j, P.b) : -1;
    }
  };
  fetch(0);
  for (int64_t j0 = 0; j0 < P.n; j0 += step) {  // workgroup-uniform
    int64_t cur[kPlanScan];
#pragma unroll
    for (int k = 0; k < kPlanScan; ++k) cur[k] = nx[k];
    if (j0 + step < P.n) fetch(j0 + step);
#pragma unroll
    for (int k = 0; k < kPlanScan; ++k) {
      if (cur[k] < 0 || cur[k] >= P.N) continue;
      const int32_t x = static_cast<int32_t>(cur[k]);
      int s = plan_hash(x, hbits);
      int32_t key = hkey[s];
      while (key != x && key != -1) {
        s = (s + 1) & (H - 1);
        key = hkey[s];
      }
      if (key == x) {
        const int64_t j = j0 + static_cast<int64_t>(k) * T + t;
        atomicAdd(&mine_ba[s], j < lo ? 1u : 0x10000u);
      }
    }
  }
  __syncthreads();
  if (i < P.n) {
    int64_t slot = -1, wnew = -1;
    if (u >= 0) {
      int below = 0, mine = 0, before = 0, after = 0;
      for (int w2 = 0; w2 < nw; ++w2) {
        const int c2 = wcnt[static_cast<size_t>(w2) * H + hs];
        mine += c2;
        if (w2 < wv) below += c2;
      }
      for (int s2 = 0; s2 < nsets; ++s2) {
        const uint32_t ba = hba[static_cast<size_t>(s2) * H + hs];
        before += static_cast<int>(ba & 0xffffu);
        after += static_cast<int>(ba >> 16);
      }
      const int c = before + mine + after;
      const int r = before + below + wrank;
      const int kept = c < P.B ? c : P.B;
      const int m = r - (c - kept);
      if (m >= 0) {
        const uint64_t x = static_cast<uint64_t>(w) + static_cast<uint64_t>(m);
        slot = static_cast<int64_t>(x % static_cast<uint64_t>(P.B));
      }
      if (r == c - 1) wnew = w + kept;
    }
    reinterpret_cast<longlong2*>(P.krec)[i] = make_longlong2(slot, wnew);
  }
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
