// The plan half of the ring update (kernel a), shared by the stand-alone ring
// kernels (tgx_ring.hip) and the plan role fused into the gather launch
// (tgx_recent.hip).
//
// A plan reads the batch's src/dst/time and writes only the ring's scratch
// (per-node counters, node lists, control words) and the caller's workspace,
// never the ring arrays, so it can run in the same launch as a gather over the
// ring.  Tickets number the entries of a node in no particular order; the
// commit ranks them by entry index.
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
// Two-launch: two cursor sets (uint64 at words 8 and 10: groups | large counts)
// and two diagnostics pairs (time flag, bad count at 16 + 2p), used by alternate
// plans.  A plan takes set p = phase_next and records it in
// phase_cur; its commit reads set phase_cur, and its workgroup 0 clears the other
// set (its plan is committed), reports and clears this plan's diagnostics and
// sets phase_next to the other set, so nothing waits for the last workgroup.
enum {
  kCtlCursor = 0, kCtlGroups = 1, kCtlTimeOk = 2, kCtlLarge = 3, kCtlBad = 4,
  kCtlFCursor = 8,  // + 2p
  kCtlPhaseNext = 12, kCtlPhaseCur = 13,
  kCtlFDiag = 16    // + 2p: time flag, + 2p + 1: bad count
};
constexpr int kCtlWords = 32;
// fields of the two-launch cursor word (every count is at most n <= 2^15)
constexpr int kFieldBits = 21;
constexpr uint64_t kFieldMask = (uint64_t(1) << kFieldBits) - 1;
enum { kFGroups = 0, kFLarge = 1 };
__host__ __device__ constexpr int field(uint64_t x, int f) {
  return static_cast<int>((x >> (f * kFieldBits)) & kFieldMask);
}

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
  int32_t* cnt;    // [N] per-node counters (zero between calls)
  int32_t* lst;    // [N, kListCap] node lists
  int32_t* ctl;    // [kCtlWords]
  int32_t* ticket; // [n] four-launch tickets; two-launch: node of every entry (-1: bad)
  int32_t* list;   // [n] four-launch lists
  int32_t* groups; // [n/2 + 1] groups
  int32_t* large;  // [n/(kListCap+1) + 1] large groups
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

// Two-launch plan of entries [block * blockDim.x, +blockDim.x) (blockDim.x a
// multiple of kWave, at most kPlanMaxThreads; every thread of the workgroup
// calls it), into cursor set phase_next.  Ticket t < kListCap stores the entry
// in lst[u][t]; the ticket-1 entry appends u to the group list, the
// ticket-kListCap entry to the large-group list.  Every entry's node goes to
// ticket[i] as int32, where the commit of a large group finds the node's
// entries.  The two wave counts are packed in one word: a workgroup prefix in
// LDS, then one cursor atomic per workgroup.
__device__ __forceinline__ void plan_block(const PlanParams& P, int64_t block, PlanLds& L) {
  const int64_t i = block * blockDim.x + threadIdx.x;
  const int wv = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  // nobody writes phase_next while a plan runs; every workgroup records the
  // same phase for the commit
  const int ph = P.ctl[kCtlPhaseNext] & 1;
  if (threadIdx.x == 0) P.ctl[kCtlPhaseCur] = ph;
  int bad;
  bool time_ok;
  const int32_t u = entry_prologue(P, i, bad, time_ok);
  const int32_t t = node_ticket(P, u, L);
  if (i < P.n) P.ticket[i] = u;
  if (t >= 0 && t < kListCap) P.lst[static_cast<int64_t>(u) * kListCap + t] = static_cast<int32_t>(i);
  const uint64_t gm = __ballot(t == 1);
  const uint64_t lm = __ballot(t == kListCap);
  if (lane == 0)
    L.wofs[wv] = (static_cast<uint64_t>(__popcll(gm)) << (kFGroups * kFieldBits)) |
                 (static_cast<uint64_t>(__popcll(lm)) << (kFLarge * kFieldBits));
  __syncthreads();
  if (threadIdx.x == 0) {
    const int nw = static_cast<int>(blockDim.x) / kWave;
    uint64_t tot = 0;
    for (int w = 0; w < nw; ++w) {
      const uint64_t c = L.wofs[w];
      L.wofs[w] = tot;
      tot += c;
    }
    L.wofs[kPlanMaxWaves] =
        tot != 0 ? atomicAdd(reinterpret_cast<unsigned long long*>(P.ctl + kCtlFCursor + 2 * ph),
                             static_cast<unsigned long long>(tot))
                 : 0;
  }
  __syncthreads();
  const uint64_t below = (uint64_t(1) << lane) - 1;
  const uint64_t at = L.wofs[kPlanMaxWaves] + L.wofs[wv];
  if (t == 1) P.groups[field(at, kFGroups) + __popcll(gm & below)] = u;
  if (t == kListCap) P.large[field(at, kFLarge) + __popcll(lm & below)] = u;
  report_diagnostics(P, bad, time_ok, kCtlFDiag + 2 * ph, kCtlFDiag + 2 * ph + 1);
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
