// Kernels (b) + (c): fused most-recent-K gather with time encoding and
// co-occurrence counts, one launch per prepared batch.
//
// Semantics (reference paths relative to the tgengine checkout):
//   * candidates of query (u, t): the CSR window of u (the last min(cnt, K)
//     entries with time < t, tgengine/core/temporal_graph.py:241-305) plus the
//     ring slots of max(u, 0) with id != -1 and time < t (_merge_overflow
//     :307-349; a padding query reads node 0's ring there, the CSR window of a
//     padding query is empty).  The V = min(#candidates, K) most recent are
//     written right-aligned in ascending time; the K - V leading positions are
//     padding (-1, 0.0, zero row, mask 0).  Equal times keep CSR-before-ring,
//     then slot order.
//   * time encoding: out_te[q,p,j] = cos(fl32(dt*w_j) [+ b_j]) with dt per
//     TGX_DT_* (tgengine/nn/time_encoding.py:55-63, tgengine/models/dygformer.py:273-279).
//   * co-occurrence for the (query 0, query 1) pair of a plan group:
//     TGX_CO_FREQ as temporal_sample.cu:453-511 plus the (B,) pair count of
//     tgengine/pipeline/__init__.py:206-219; TGX_CO_DYGFORMER as
//     tgengine/models/dygformer.py:71-87 on the 1+K sequences with the node first.
//
// Mapping.  One wavefront per query, `group` queries per workgroup (a plan group
// puts a (src, dst) pair in one workgroup for the co-occurrence counts).  Lane s
// loads ring slot s (with its feature row when the row is at most 64 bytes, in
// the same memory round trip) and the node's write position.  Ranking:
//   * fast path (no CSR candidates): a ring is written oldest-to-newest from slot
//     write_pos % B on, so when the filled slots are exactly the last ones in that
//     write order and their times strictly increase along it, a candidate's rank
//     is its write-order distance from the oldest filled slot (one shuffle and
//     two ballots verify the premise);
//   * otherwise the candidates go to an LDS list (CSR window first, then ring
//     slots) and each is ranked by counting earlier (time, index) entries.
// The lane holding a selected candidate writes its id / time / mask at output
// position K - V + rank - drop; feature rows then move to their positions by
// lane shuffles (small rows) or 16-byte loads/stores spread over the wave, and
// the K x d_t encodings stream out as float4 nontemporal stores with the pad
// rows (DyGFormer dt mode) written as zeros without evaluating a cosine.  The
// cosine of the exact fp32 argument x is v_cos_f32 of the revolution fraction of
// x (tgx_cos.h): 6 VALU per element while every argument of the wave is below
// 2^29, a table-driven exact reduction otherwise.
#include "tgx_internal.h"
#include <hip/hip_ext.h>

#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "tgx_cos.h"
#include "tgx_ring_plan.h"

namespace tgx {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Params {
  // ring
  int64_t N;
  int B;  // 0 when there is no ring
  int b_pow2;
  const int32_t* r_ids;
  const double* r_times;
  const uint8_t* r_feats;
  const int64_t* r_eids;
  const int64_t* r_wp;
  // csr
  int has_csr;
  const int64_t* c_off;
  const int32_t* c_ids;
  const double* c_times;
  const uint8_t* c_feats;
  const int64_t* c_eids;
  // queries
  const int64_t* nodes;
  const double* qtimes;
  int ngroups;
  const void* gn[TGX_MAX_QUERY_GROUPS];
  const uint8_t* gv[TGX_MAX_QUERY_GROUPS];  // per-query validity or null
  int gi32[TGX_MAX_QUERY_GROUPS];           // int32 node ids
  const double* gt[TGX_MAX_QUERY_GROUPS];
  int64_t goff[TGX_MAX_QUERY_GROUPS + 1];
  int gdiv[TGX_MAX_QUERY_GROUPS];
  int64_t Q;
  int K;
  const int32_t* plan;
  int G;
  // outputs
  int64_t row_bytes;
  int nch;  // row_bytes / VEC
  int32_t* o_ids;
  double* o_times;
  uint8_t* o_feats;
  uint8_t* o_mask;
  int64_t* o_eids;
  int d_t;
  const float* te_w;
  const float* te_b;
  int dt_mode;
  float* o_te;
  int te_vec4;
  int co_mode;
  int32_t* co_a;
  int32_t* co_c;
  float* co_pair;
  int32_t* status;
  // LDS layout: weights (te_bytes), then one wave_bytes region per wavefront
  int te_bytes;
  int wave_bytes;
  int cand_cap;
  int off_cid, off_code, off_pcode, off_pdt, off_pid, off_pt, off_pe, off_tab;
  // work decomposition: m queries per wavefront in sub-groups of 2^lg_bp lanes
  int m, lg_bp;
  // FastDiv multipliers of K, d_t / 4, d_t and nch
  uint32_t fd_k, fd_q, fd_d, fd_c;
  // wavefronts per query (m == 1), each writing every split-th output chunk: the
  // count itself for tiled launches, its log2 for the others (each copy of the
  // kernel divides or shifts, whichever measured faster there)
  int split;
  // fused ring plan: workgroups [0, plan_blocks) plan the caller's next batch
  PlanParams pl;
  int plan_blocks;
  int plan_mode;  // TGX_PLAN_*
  // event-major plan over b events: query slot j of event g is
  // b * before_j + g * per_j + index_j, with 12 bits per slot in ev_code
  // (before_j: queries per event of the earlier query groups, per_j: of this
  // group, index_j: the slot's index among them)
  uint64_t ev_code[2];
  int64_t ev_b;
  // queries of the query groups after the event groups: from ev_tail on, G
  // consecutive ones per workgroup, workgroups [ev_b, ...) of the plan
  int64_t ev_tail;
  // |dt| below which no encoding argument reaches kRevArg (0: none is known)
  float te_dt_small;
  double c_tmax;  // largest non-NaN CSR time (+inf: unknown)
  int wg_parts;   // csr_split: workgroups per query (1: a workgroup holds whole queries)
  int te_nt;      // csr_split: nontemporal encoding stores (rows of at least kNtRowBytes)
};

template <int VEC>
struct Vec;
template <>
struct Vec<16> {
  using T = u32x4;
};
template <>
struct Vec<4> {
  using T = uint32_t;
};
template <>
struct Vec<2> {
  using T = uint16_t;
};

__constant__ double kRevTableDev[][2] = {TGX_REV_TABLE_ROWS};

// cos(x) as v_cos_f32 of the fp32-rounded revolution fraction (tgx_cos.h):
// cos_small for |x| < kRevArg, cos_full for every fp32 x
__device__ __forceinline__ float cos_small(float x) {
  return __builtin_amdgcn_cosf(static_cast<float>(rev_frac_small(x)));
}
__device__ __forceinline__ float cos_full(float x) {
  return __builtin_amdgcn_cosf(static_cast<float>(rev_frac(x, kRevTableDev)));
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ u32x4 shfl_v(u32x4 x, int src) {
  u32x4 r;
  r[0] = __shfl(x[0], src);
  r[1] = __shfl(x[1], src);
  r[2] = __shfl(x[2], src);
  r[3] = __shfl(x[3], src);
  return r;
}

// Output stores.  Small-row launches write with ordinary stores (the encodings
// then stream out of L2 at a higher rate); large-row launches, whose row copy
// already streams, use nontemporal stores (measured faster for both shapes).
template <bool NT, typename T>
__device__ __forceinline__ void put(T* p, const T& v) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

// wavefronts per workgroup, the kernel's launch bound (512 threads)
constexpr int kMaxWaves = 8;

// queries of a launch above which small-row queries are packed several per wave
// (about the wave slots of one MI355X: 256 CUs x 4 SIMDs x 8)
constexpr int64_t kPackMinQueries = 8192;

// output bytes of one query below which its waves are not split further
constexpr int64_t kSplitBytes = 8192;

// waves of a launch up to which a small launch's queries are split further (half
// the device's wave slots: 600 queries ran faster at 4 waves each than at 8)
constexpr int64_t kSplitMaxWaves = 4096;

// compute units of one MI355X (the LDS residency bound of the split rule)
constexpr int64_t kDeviceCUs = 256;

// row chunks each lane loads before storing them (large-row copy)
constexpr int kCopyDepth = 4;
// csr_split: a query split over more wavefronts than this spreads them over
// workgroups of this many (Reddit's 600 queries x 8 waves: 12.3 -> 11.7 us, LastFM's
// 31.5 -> 30.0 us; 2 or 1 wave per workgroup measured no better)
constexpr int kSplitGroupWaves = 4;
// csr_split: rows of at least this many bytes stream, and the encodings beside
// them go out as nontemporal stores
constexpr int64_t kNtRowBytes = 64;
// node ids per thread and step of the ring plan's batch scan when the plan runs
// in a gather launch (its registers stay within the gather's)
constexpr int kFusedPlanScan = 4;

// x / n for x * n < 2^32 (n >= 1): one multiply-high by ceil(2^32 / n)
struct FastDiv {
  uint32_t n, m;
  // the multiplier of divisor n (computed on the host: a division is tens of
  // VALU instructions on the device)
  __host__ __device__ static constexpr uint32_t magic(uint32_t n) {
    return n > 1 ? 0xffffffffu / n + 1u : 0u;
  }
  __device__ FastDiv(uint32_t n_, uint32_t m_) : n(n_), m(m_) {}
  __device__ __forceinline__ uint32_t div(uint32_t x) const { return n > 1 ? __umulhi(x, m) : x; }
};

// smallest i in [lo, hi] with i == hi or t[i] >= q (t ascending); wave-uniform result
template <bool CLAMP>
__device__ __forceinline__ int64_t wave_lower_bound(const double* __restrict__ t, int64_t lo,
                                                    int64_t hi, double q, int lane) {
  while (hi - lo > kWave) {
    const int64_t step = (hi - lo + kWave - 1) / kWave;
    const int64_t pos0 = lo + static_cast<int64_t>(lane + 1) * step - 1;
    int64_t pc, nl;
    if constexpr (CLAMP) {
      // probes clamped to the window's last entry, so they stay in order and the
      // top lane reads t[hi - 1]: a query after the whole window ends in one round
      const int64_t pos = pos0 < hi ? pos0 : hi - 1;
      const int c = __popcll(__ballot(t[pos] < q));
      pc = lo + static_cast<int64_t>(c + 1) * step - 1;
      nl = lo + static_cast<int64_t>(c) * step;
      nl = nl < hi ? nl : hi;  // every probe below q: lo = hi, and the search ends
    } else {
      const bool pr = pos0 < hi && t[pos0] < q;
      const int c = __popcll(__ballot(pr));
      pc = lo + static_cast<int64_t>(c + 1) * step - 1;
      nl = lo + static_cast<int64_t>(c) * step;
    }
    lo = nl;
    hi = pc < hi ? pc : hi;
  }
  const int64_t pos = lo + lane;
  const bool pr = pos < hi && t[pos] < q;
  return lo + __popcll(__ballot(pr));
}

// wave_lower_bound<true> run by every sub-group of Bp = 2^lg lanes at once on
// its own query (lo, hi and q uniform within the sub-group h; active: whether
// the sub-group searches at all): Bp-ary rounds with probes clamped to hi - 1,
// until at most Bp entries are left.  Returns the first index in [lo, hi] whose
// time is not below q.
__device__ __forceinline__ int64_t subgroup_lower_bound(const double* __restrict__ t, int64_t lo, int64_t hi,
                                                        double q, bool active, int sl, int h, int lg) {
  const int Bp = 1 << lg;
  const uint64_t submask = Bp == kWave ? ~uint64_t(0) : ((uint64_t(1) << Bp) - 1);
  while (true) {
    const bool more = active && hi - lo > Bp;
    if (__ballot(more) == 0) break;  // wave-uniform
    int64_t step = 0;
    bool pr = false;
    if (more) {
      step = (hi - lo + Bp - 1) >> lg;
      const int64_t pos0 = lo + static_cast<int64_t>(sl + 1) * step - 1;
      pr = t[pos0 < hi ? pos0 : hi - 1] < q;
    }
    const uint64_t below = (__ballot(more && pr) >> (h << lg)) & submask;
    if (more) {
      const int64_t c = __popcll(below);
      const int64_t pc = lo + (c + 1) * step - 1;
      const int64_t nl = lo + c * step;
      lo = nl < hi ? nl : hi;
      hi = pc < hi ? pc : hi;
    }
  }
  const int64_t pos = lo + sl;
  const bool pr = active && pos < hi && t[pos] < q;
  return lo + __popcll((__ballot(pr) >> (h << lg)) & submask);
}

// Query j of plan group g (-1: none).  Event-major groups: group g is event g,
// and its j-th query is, for each query group in order, one of that group's
// times_per queries of event g; every query group holds b x times_per queries,
// so the query is b * before + g * per + index with the slot's three small
// constants decoded from ev_code by shifts.
__device__ __forceinline__ int64_t query_of(const Params& P, int64_t g, int j) {
  if (j >= P.G) return -1;
  if (P.plan_mode == TGX_PLAN_EVENTS) {
    if (g >= P.ev_b) {
      const int64_t q = P.ev_tail + (g - P.ev_b) * P.G + j;
      return q < P.Q ? q : -1;
    }
    const uint64_t w = j < 5 ? P.ev_code[0] >> (12 * j) : P.ev_code[1] >> (12 * (j - 5));
    const int before = static_cast<int>(w & 15u), per = static_cast<int>((w >> 4) & 15u);
    return P.ev_b * before + g * per + static_cast<int>((w >> 8) & 15u);
  }
  const int64_t slot = g * P.G + j;
  const int64_t q = P.plan != nullptr ? static_cast<int64_t>(P.plan[slot]) : slot;
  return (q >= 0 && q < P.Q) ? q : -1;
}

// node and time of query q, and whether it is a query at all (a group's
// validity array can turn it into padding output only); the query group is
// chosen with compares against the group offsets (constant indices only, so the
// arguments stay in registers)
__device__ __forceinline__ void query_load(const Params& P, int64_t q, int64_t& node, double& qt,
                                           bool& valid) {
  valid = true;
  if (P.ngroups == 0) {
    node = P.nodes[q];
    qt = P.qtimes[q];
    return;
  }
  const void* np = P.gn[0];
  const double* tp = P.gt[0];
  const uint8_t* vp = P.gv[0];
  int64_t off = 0;
  int div = P.gdiv[0];
  int i32 = P.gi32[0];
#pragma unroll
  for (int g = 1; g < TGX_MAX_QUERY_GROUPS; ++g) {
    if (g < P.ngroups && q >= P.goff[g]) {
      np = P.gn[g];
      tp = P.gt[g];
      vp = P.gv[g];
      off = P.goff[g];
      div = P.gdiv[g];
      i32 = P.gi32[g];
    }
  }
  const int64_t l = q - off;
  node = i32 ? static_cast<int64_t>(static_cast<const int32_t*>(np)[l]) : static_cast<const int64_t*>(np)[l];
  qt = tp[div == 1 ? l : static_cast<int64_t>(static_cast<uint32_t>(l) / static_cast<uint32_t>(div))];
  if (vp != nullptr) valid = vp[l] != 0;
}

__device__ __forceinline__ int64_t query_node(const Params& P, int64_t q) {
  int64_t node;
  double qt;
  bool valid;
  query_load(P, q, node, qt, valid);
  return node;
}

// Time encodings of np consecutive output rows starting at row r0 (the wave's
// queries are consecutive): out_te[r0 + gp, :] from pdt[gp]; a DyGFormer pad
// (pcode < 0) encodes to zeros without evaluating a cosine.
template <bool BIG, bool NT>
__device__ __forceinline__ void encode_rows(const Params& P, int64_t r0, int np, const int32_t* pcode,
                                            const float* pdt, const float* s_w, const float* s_b,
                                            int start, int stride) {
  const int d_t = P.d_t;
  const bool dyg = P.dt_mode == TGX_DT_DYGFORMER;
  const bool has_b = P.te_b != nullptr;
  if (P.te_vec4) {
    const int nq = d_t / 4;
    const int total = np * nq;
    const FastDiv dq(nq, P.fd_q);
    const f32x4* w4 = reinterpret_cast<const f32x4*>(s_w);
    const f32x4* b4 = reinterpret_cast<const f32x4*>(s_b);
    f32x4* o4 = reinterpret_cast<f32x4*>(P.o_te) + r0 * nq;
    for (int idx = start; idx < total; idx += stride) {
      const int gp = static_cast<int>(dq.div(idx));
      const int c = idx - gp * nq;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      if (!dyg || pcode[gp] >= 0) {
        f32x4 a = pdt[gp] * w4[c];
        if (has_b) a = a + b4[c];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = BIG ? cos_full(a[j]) : cos_small(a[j]);
      }
      put<NT>(o4 + idx, o);
    }
  } else {
    const int total = np * d_t;
    const FastDiv dd(d_t, P.fd_d);
    float* out = P.o_te + r0 * d_t;
    for (int idx = start; idx < total; idx += stride) {
      const int gp = static_cast<int>(dd.div(idx));
      const int j = idx - gp * d_t;
      float o = 0.f;
      if (!dyg || pcode[gp] >= 0) {
        float a = pdt[gp] * s_w[j];
        if (has_b) a = a + s_b[j];
        o = BIG ? cos_full(a) : cos_small(a);
      }
      out[idx] = o;
    }
  }
}

// Co-occurrence counts of one (query a, query c) pair by one wavefront; A and Cc
// are the K neighbour ids of the two queries (LDS).  Output row g.
__device__ __forceinline__ void co_occurrence_pair(const Params& P, int64_t g, int64_t qa, int64_t qc,
                                                   const int32_t* A, const int32_t* Cc, int lane) {
  const int K = P.K;
  if (P.co_mode == TGX_CO_FREQ && K <= kWave / 2) {
    // both sides in one pass: lanes [0, 32) take A's positions, lanes [32, 64) C's
    const int side = lane >> 5;
    const int i = lane & 31;
    const int32_t x = i < K ? (side == 0 ? A[i] : Cc[i]) : -1;
    int na = 0, nc = 0;
    if (x != -1) {
      for (int j = 0; j < K; ++j) {
        na += A[j] == x;
        nc += Cc[j] == x;
      }
    }
    if (i < K) {
      int32_t* out = side == 0 ? P.co_a : P.co_c;
      out[(g * K + i) * 2 + 0] = na;
      out[(g * K + i) * 2 + 1] = nc;
    }
    const int pc = __popcll(__ballot(side == 0 && i < K && x != -1 && nc > 0));
    if (lane == 0 && P.co_pair != nullptr) P.co_pair[g] = static_cast<float>(pc);
    return;
  }
  if (P.co_mode == TGX_CO_FREQ) {
    for (int side = 0; side < 2; ++side) {
      const int32_t* X = side == 0 ? A : Cc;
      int32_t* out = side == 0 ? P.co_a : P.co_c;
      int pc = 0;
      for (int i0 = 0; i0 < K; i0 += kWave) {
        const int i = i0 + lane;
        int32_t x = -1;
        int na = 0, nc = 0;
        if (i < K) {
          x = X[i];
          if (x != -1) {
            for (int j = 0; j < K; ++j) {
              na += A[j] == x;
              nc += Cc[j] == x;
            }
          }
          out[(g * K + i) * 2 + 0] = na;
          out[(g * K + i) * 2 + 1] = nc;
        }
        pc += __popcll(__ballot(i < K && x != -1 && nc > 0));
      }
      if (side == 0 && lane == 0 && P.co_pair != nullptr) P.co_pair[g] = static_cast<float>(pc);
    }
    return;
  }
  // DyGFormer counts on A' = [node_a] ++ A, C' = [node_c] ++ C (length K+1)
  const int32_t na0 = static_cast<int32_t>(query_node(P, qa));
  const int32_t nc0 = static_cast<int32_t>(query_node(P, qc));
  const int L = K + 1;
  if (P.co_pair != nullptr) {
    // (B,) count over the K sequences, as in FREQ mode
    int pc = 0;
    for (int i0 = 0; i0 < K; i0 += kWave) {
      const int i = i0 + lane;
      bool hit = false;
      if (i < K && A[i] != -1)
        for (int j = 0; j < K && !hit; ++j) hit = Cc[j] == A[i];
      pc += __popcll(__ballot(hit));
    }
    if (lane == 0) P.co_pair[g] = static_cast<float>(pc);
  }
  for (int side = 0; side < 2; ++side) {
    int32_t* out = side == 0 ? P.co_a : P.co_c;
    for (int i = lane; i < L; i += kWave) {
      const int32_t ai = i == 0 ? na0 : A[i - 1];
      const int32_t ci = i == 0 ? nc0 : Cc[i - 1];
      int f0 = 0, f1 = 0;
      if (side == 0) {
        if (ai != -1) {
          for (int j = 0; j < L; ++j) {
            const int32_t aj = j == 0 ? na0 : A[j - 1];
            const int32_t cj = j == 0 ? nc0 : Cc[j - 1];
            f0 += aj == ai;
            f1 += (aj == ci) && (cj != -1);
          }
        }
      } else {
        if (ci != -1) {
          for (int j = 0; j < L; ++j) {
            const int32_t aj = j == 0 ? na0 : A[j - 1];
            const int32_t cj = j == 0 ? nc0 : Cc[j - 1];
            f0 += (cj == ai) && (aj != -1);
            f1 += cj == ci;
          }
        }
      }
      out[(g * L + i) * 2 + 0] = f0;
      out[(g * L + i) * 2 + 1] = f1;
    }
  }
}

// One wavefront per tile of queries.  No plan: a tile is m = 64/Bp consecutive
// queries (sub-group h = lanes h*Bp .. h*Bp+Bp-1 takes query h, Bp >= B); with
// a plan: m = 1 and the workgroup is the plan group, wave j taking query j.
// Every load of the wave (queries, ring slots and small feature rows, CSR
// windows, edge ids) is issued and consumed before its first global store:
// gfx9 counts vector loads and stores in one in-order vmcnt, so a load behind
// stores would wait for their completion.  With at most one wave per SIMD slot
// for the whole grid the gathers all run up front and the stores then stream.
// Waves-per-SIMD target: 8 for the event- and list-plan kernels with rows through
// memory, whose bandwidth needs every resident wave (plan-group workgroups of 6
// waves fit 5 per CU at 8, 4 at 7; without the target C5's gather took 200 us
// instead of 176); none for the small-row kernels and the tiled 16-byte-chunk
// kernel, where forcing 8 capped the scalar registers and spilled them into their
// own code (the tiled one: 8.56 -> 7.74 us on C1 and 367 -> 356 us on C4 without
// it), while the 7 the registers allow still hold their grids.
template <int VEC, int NREG, bool TILES>
constexpr int kWavesPerEu = NREG > 0 || (TILES && VEC == 16) ? 1 : 8;

// TILES: the launch's plan mode is TGX_PLAN_TILES (no event or list plan, so no
// co-occurrence); that copy of the kernel carries none of their code, which
// shortens its start-up
template <int VEC, int NREG, bool TILES>
__global__ __launch_bounds__(kMaxWaves * kWave) __attribute__((amdgpu_waves_per_eu(kWavesPerEu<VEC, NREG, TILES>)))
void recent_fused(Params P) {
  using VT = typename Vec<VEC>::T;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  if (static_cast<int>(blockIdx.x) < P.plan_blocks) {
    // the plan reads the ring's write positions and writes only its scratch and
    // the workspace, never the arrays gathered here
    plan_block_ordered<kFusedPlanScan>(P.pl, blockIdx.x, smem);
    return;
  }
  const int64_t g = static_cast<int64_t>(blockIdx.x) - P.plan_blocks;
  const int K = P.K;
  const int B = P.B;
  const int C = P.cand_cap;
  const int m = P.m;
  const int lg = P.lg_bp;
  const int Bp = 1 << lg;
  const int h = lane >> lg;
  const int sl = lane & (Bp - 1);
  const uint64_t submask = Bp == kWave ? ~uint64_t(0) : ((uint64_t(1) << Bp) - 1);
  const bool dyg = P.dt_mode == TGX_DT_DYGFORMER;

  float* s_w = reinterpret_cast<float*>(smem);
  float* s_b = s_w + (P.te_bytes / 8);
  for (int i = threadIdx.x; i < P.d_t; i += blockDim.x) {
    s_w[i] = P.te_w[i];
    s_b[i] = P.te_b != nullptr ? P.te_b[i] : 0.0f;
  }
  __syncthreads();
  uint8_t* wb = smem + P.te_bytes + static_cast<size_t>(wv) * P.wave_bytes;
  double* ct = reinterpret_cast<double*>(wb);                       // [m][C] candidates
  int32_t* cid = reinterpret_cast<int32_t*>(wb + P.off_cid);
  int32_t* ccode = reinterpret_cast<int32_t*>(wb + P.off_code);
  int32_t* pcode = reinterpret_cast<int32_t*>(wb + P.off_pcode);  // [m][K] slot, B + CSR index, -1
  float* pdt = reinterpret_cast<float*>(wb + P.off_pdt);           // [m][K] dt
  int32_t* pid = reinterpret_cast<int32_t*>(wb + P.off_pid);       // [m][K] id
  double* pt = reinterpret_cast<double*>(wb + P.off_pt);           // [m][K] time
  int64_t* tq = reinterpret_cast<int64_t*>(wb + P.off_tab);        // [m] query (-1 = none)
  int64_t* tur = tq + m;                                            // [m] ring row
  int64_t* tcb = tur + m;                                           // [m] CSR window start
  int64_t* pe = reinterpret_cast<int64_t*>(wb + P.off_pe);         // [m][K] edge id

  // ---- the wave's queries: query slot wv / split of the workgroup; the split
  // waves of one query repeat its (cheap) gather and share its outputs ----
  const int split = TILES ? P.split : 1 << P.split;
  const int qs = TILES ? wv / split : wv >> P.split;
  const int part = TILES ? wv - qs * split : wv & (split - 1);
  int64_t q;
  if (!TILES && P.plan_mode != TGX_PLAN_TILES) {
    q = query_of(P, g, qs);
  } else {
    const int64_t t = g * (blockDim.x / kWave / split) + qs;
    q = t * m + h;
    if (q >= P.Q) q = -1;
  }
  int64_t node = -1;
  double qt = 0.0;
  bool qvalid = true;
  if (q >= 0) query_load(P, q, node, qt, qvalid);
  const bool bad = q >= 0 && qvalid && node >= P.N;
  if (bad && sl == 0 && part == 0 && P.status != nullptr) atomicAdd(&P.status[TGX_ST_BAD_QUERY_NODE], 1);
  const int64_t ur = node < 0 ? 0 : node;
  const bool live = q >= 0 && qvalid && !bad;

  // ---- ring slot sl of query h, its feature row (NREG > 0) and write position ----
  int32_t rid = -1;
  double rt = 0.0;
  int64_t wp = 0;
  VT rows[NREG > 0 ? NREG : 1];
#pragma unroll
  for (int k = 0; k < (NREG > 0 ? NREG : 1); ++k) rows[k] = VT{};
  if (live && B > 0) {
    // the slot's id and time and the write position first: the rank waits for
    // them, and loads complete in order, so the rows (NREG > 0) come last
    if (sl < B) {
      rid = P.r_ids[ur * B + sl];
      rt = P.r_times[ur * B + sl];
    }
    if (P.r_wp != nullptr) wp = P.r_wp[ur];
    if constexpr (NREG > 0) {
      if (sl < B) {
        const VT* src = reinterpret_cast<const VT*>(P.r_feats + (ur * B + sl) * P.row_bytes);
#pragma unroll
        for (int k = 0; k < NREG; ++k)
          if (k < P.nch) rows[k] = src[k];
      }
    }
  }

  // ---- CSR windows: a 64-ary search per query of the wave, all lanes ----
  int ncsr = 0;
  int64_t cbase = 0;
  if (P.has_csr) {
    for (int hh = 0; hh < m; ++hh) {
      const int64_t nh = __shfl(node, hh << lg);
      const double th = __shfl(qt, hh << lg);
      const int lh = __shfl(static_cast<int>(live), hh << lg);
      if (lh && nh >= 0) {
        const int64_t s0 = P.c_off[nh];
        const int64_t s1 = P.c_off[nh + 1];
        const int64_t cnt = wave_lower_bound<TILES>(P.c_times, s0, s1, th, lane) - s0;
        const int take = static_cast<int>(cnt < K ? cnt : K);
        if (h == hh) {
          ncsr = take;
          cbase = s0 + cnt - take;
        }
      }
    }
    for (int j = sl; j < ncsr; j += Bp) {
      ct[h * C + j] = P.c_times[cbase + j];
      cid[h * C + j] = P.c_ids[cbase + j];
      ccode[h * C + j] = B + j;
    }
  }
  const bool v = live && sl < B && rid != -1 && rt < qt;
  const uint64_t mine = (__ballot(v) >> (h << lg)) & submask;
  const int ncand = ncsr + __popcll(mine);
  const int V = ncand < K ? ncand : K;
  const int drop = ncand - V;
  if (sl == 0) {
    tq[h] = q;
    tur[h] = ur;
    tcb[h] = cbase;
  }

  // ---- rank into LDS positions ----
  bool lane_big = false;
  auto emit = [&](int p, int32_t id, double t, int code) {
    const int pp = h * K + p;
    const float dt = dyg ? static_cast<float>(qt) - static_cast<float>(t) : static_cast<float>(qt - t);
    pdt[pp] = dt;
    pt[pp] = t;
    pcode[pp] = code;
    pid[pp] = id;
    lane_big |= (!dyg || code >= 0) && !(fabsf(dt) < P.te_dt_small);
  };
  // fast path: no CSR candidates, and the filled slots are the newest ones in
  // write order (oldest = slot write_pos % B) with strictly increasing times;
  // then a candidate's rank is its write-order distance from the oldest filled slot
  bool broken = true;
  int order = 0;
  const bool try_fast = live && ncsr == 0 && B > 0 && P.r_wp != nullptr;
  if (try_fast) {
    const int w = P.b_pow2 ? static_cast<int>(wp & (B - 1)) : static_cast<int>(wp % B);
    order = sl - w < 0 ? sl - w + B : sl - w;
    const uint64_t filled = (__ballot(sl < B && rid != -1) >> (h << lg)) & submask;
    const int empty = B - __popcll(filled);
    const int nxt = sl + 1 == B ? 0 : sl + 1;
    const double tn = __shfl(rt, (h << lg) + nxt);
    broken = sl < B && (((rid != -1) != (order >= empty)) || (rid != -1 && order < B - 1 && !(rt < tn)));
    order -= empty;
  }
  const bool fast = try_fast && ((__ballot(broken) >> (h << lg)) & submask) == 0;
  if (q >= 0) {
    if (fast) {
      if (v && order >= drop) emit(K - V + (order - drop), rid, rt, sl);
    } else if (v) {
      const int at = h * C + ncsr + __popcll(mine & ((uint64_t(1) << sl) - 1));
      ct[at] = rt;
      cid[at] = rid;
      ccode[at] = sl;
    }
  }
  wave_sync();
  if (q >= 0) {
    if (!fast) {
      // counting rank by (time, CSR-before-ring, candidate index).  The CSR
      // window is time-ascending with ties in CSR order, so CSR entry c has
      // exactly c such predecessors among the CSR entries and only the ring
      // candidates need counting; a ring candidate counts them all
      for (int c = sl; c < ncand; c += Bp) {
        const double tc = ct[h * C + c];
        int r = c < ncsr ? c : 0;
        for (int c0 = c < ncsr ? ncsr : 0; c0 < ncand; c0 += 4) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int c2 = c0 + u;
            if (c2 < ncand) {
              const double t2 = ct[h * C + c2];
              r += (t2 < tc) || (t2 == tc && c2 < c);
            }
          }
        }
        if (r >= drop) emit(K - V + (r - drop), cid[h * C + c], tc, ccode[h * C + c]);
      }
    }
    for (int p = sl; p < K - V; p += Bp) emit(p, -1, 0.0, -1);
  } else {
    for (int p = sl; p < K; p += Bp) {
      pcode[h * K + p] = -1;
      pid[h * K + p] = -1;
    }
  }
  const bool te_big = __ballot(lane_big) != 0;
  wave_sync();

  // the wave's valid queries are consecutive from q0: output row q0*K + gp for
  // wave position gp = h*K + p < np
  const int64_t q0 = tq[0];
  int nvalid = 0;
  for (int hh = 0; hh < m; ++hh) nvalid += tq[hh] >= 0 ? 1 : 0;
  if (q0 < 0) nvalid = 0;
  const int np = nvalid * K;
  const int64_t r0 = q0 * K;
  const FastDiv dk(K, P.fd_k);
  const int ostart = part * kWave + lane;  // this wave's share of the output chunks
  const int ostride = split * kWave;

  // ---- edge ids into LDS (loads, before any store) ----
  if (P.o_eids != nullptr) {
    for (int gp = lane; gp < np; gp += kWave) {
      const int hh = static_cast<int>(dk.div(gp));
      const int code = pcode[gp];
      int64_t e = -1;
      if (code >= 0 && code < B)
        e = P.r_eids != nullptr ? P.r_eids[tur[hh] * B + code] : -1;
      else if (code >= B)
        e = P.c_eids != nullptr ? P.c_eids[tcb[hh] + (code - B)] : -1;
      pe[gp] = e;
    }
  }

  auto store_te = [&]() {
  // ---- time encoding ----
  if (P.d_t > 0 && np > 0) {
    if (te_big)
      encode_rows<true, (NREG == 0)>(P, r0, np, pcode, pdt, s_w, s_b, ostart, ostride);
    else
      encode_rows<false, (NREG == 0)>(P, r0, np, pcode, pdt, s_w, s_b, ostart, ostride);
  }

  };
  auto store_feats = [&]() {
  // ---- feature rows: np rows x nch chunks of VEC bytes, one flat run ----
  if (P.o_feats != nullptr && P.row_bytes > 0) {
    const int nch = P.nch;
    const int total = np * nch;
    const FastDiv dv(nch, P.fd_c);
    VT* of = reinterpret_cast<VT*>(P.o_feats) + r0 * nch;
    if constexpr (NREG > 0) {
      // ring rows come from the lanes that loaded them, CSR rows from memory;
      // every lane takes part in every shuffle
      for (int b0 = part * kWave; b0 < total; b0 += ostride) {
        const int idx = b0 + lane;
        int gp = 0, c = 0, code = -1, hh = 0;
        if (idx < total) {
          gp = static_cast<int>(dv.div(idx));
          c = idx - gp * nch;
          hh = static_cast<int>(dk.div(gp));
          code = pcode[gp];
        }
        const int srcl = (code >= 0 && code < B) ? (hh << lg) + code : lane;
        VT val = VT{};
#pragma unroll
        for (int k = 0; k < NREG; ++k) {
          const VT x = shfl_v(rows[k], srcl);
          if (k == c) val = x;
        }
        if (idx < total) {
          if (code < 0)
            val = VT{};
          else if (code >= B)
            val = reinterpret_cast<const VT*>(P.c_feats + (tcb[hh] + (code - B)) * P.row_bytes)[c];
          put<false>(of + idx, val);
        }
      }
    } else {
      // the event- and list-plan copies (co-occurrence launches: C2's 200-event
      // batches) load 8 chunks per lane before storing them, the tiled ones 4 (8 made
      // C2's gather 12.95 -> 12.22 us and C5's 1% faster, C1's 8.3 -> 8.9 and C4's
      // 367 -> 381 us slower)
      constexpr int kDepth = TILES ? kCopyDepth : 2 * kCopyDepth;
      for (int idx0 = part * kWave; idx0 < total; idx0 += kDepth * ostride) {
        VT v4[kDepth];
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
          const int idx = idx0 + u * ostride + lane;
          v4[u] = VT{};
          if (idx < total) {
            const int gp = static_cast<int>(dv.div(idx));
            const int c = idx - gp * nch;
            const int hh = static_cast<int>(dk.div(gp));
            const int code = pcode[gp];
            if (code >= 0) {
              const uint8_t* src = code < B ? P.r_feats + (tur[hh] * B + code) * P.row_bytes
                                            : P.c_feats + (tcb[hh] + (code - B)) * P.row_bytes;
              v4[u] = reinterpret_cast<const VT*>(src)[c];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
          const int idx = idx0 + u * ostride + lane;
          if (idx < total) put<true>(of + idx, v4[u]);
        }
      }
    }
  }

  };
  auto store_ids = [&]() {
  // ---- ids / times / mask / edge ids ----
  for (int gp = ostart; gp < np; gp += ostride) {
    const int64_t o = r0 + gp;
    P.o_ids[o] = pid[gp];
    P.o_times[o] = pt[gp];
    P.o_mask[o] = pcode[gp] >= 0 ? 1 : 0;
    if (P.o_eids != nullptr) P.o_eids[o] = pe[gp];
  }

  };
  // Store order: with register-held rows there is nothing left to load, so the
  // bulk (the encodings) goes first; with large rows the row copy loads first,
  // before any encoding store can hold its loads back in vmcnt.
  if constexpr (NREG > 0) {
    store_te();
    store_feats();
  } else {
    store_feats();
    store_te();
  }
  store_ids();

  // ---- co-occurrence of the plan group's (query 0, query 1) pair ----
  if (!TILES && P.co_mode != TGX_CO_NONE) {
    __syncthreads();
    // workgroups from ev_b on (an event-major plan's tail) hold no pair
    const int64_t qa = g < P.ev_b ? query_of(P, g, 0) : -1;
    const int64_t qc = query_of(P, g, 1);
    if (qa >= 0 && qc >= 0 && wv == 0) {
      const int32_t* A = reinterpret_cast<const int32_t*>(smem + P.te_bytes + P.off_pid);
      const int32_t* Cc = reinterpret_cast<const int32_t*>(smem + P.te_bytes +
                                                          static_cast<size_t>(split) * P.wave_bytes + P.off_pid);
      co_occurrence_pair(P, g, qa, qc, A, Cc, lane);
    }
  }
}

// Ring-less tiled gather over a frozen CSR for K <= 64 with rows of at most NREG
// 16-byte chunks (NREG = 0: no feature rows asked for).  Sub-group h of Bp =
// 2^lg_bp >= K lanes takes query h of the wave's m = 64 / Bp consecutive
// queries, and lane sl < K owns output position sl.  With the query's CSR
// offsets in, each lane loads the entry that the window's last K would put at
// its position (time, id, row, edge id).  When the query comes after the whole
// window (its last time is below the query time; NaN times sort last, so the
// window then holds none), those entries are the answer, as the search would
// find: three dependent round trips (query, offsets, entries) before the
// stores, against five for recent_fused's search, staging and row copy.
// Otherwise the search goes on from a first Bp-ary round whose probes went out
// with those loads (a window of more than Bp entries and a query time not after
// the CSR's last one: max_time), the wave searching what is left of each such
// query's window (wave_lower_bound, as recent_fused), and the answer's entries
// are reloaded.
template <int NREG>
__global__ __launch_bounds__(kMaxWaves * kWave) void csr_window(Params P) {
  using VT = u32x4;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int K = P.K;
  const int m = P.m;
  const int lg = P.lg_bp;
  const int h = lane >> lg;
  const int sl = lane & ((1 << lg) - 1);
  const bool dyg = P.dt_mode == TGX_DT_DYGFORMER;

  float* s_w = reinterpret_cast<float*>(smem);
  float* s_b = s_w + (P.te_bytes / 8);
  if (P.d_t > 0) {  // launch-uniform
    for (int i = threadIdx.x; i < P.d_t; i += blockDim.x) {
      s_w[i] = P.te_w[i];
      s_b[i] = P.te_b != nullptr ? P.te_b[i] : 0.0f;
    }
    __syncthreads();
  }
  uint8_t* wb = smem + P.te_bytes + static_cast<size_t>(wv) * P.wave_bytes;
  int32_t* pcode = reinterpret_cast<int32_t*>(wb);        // [m][K] 0 entry, -1 pad
  float* pdt = reinterpret_cast<float*>(wb + P.off_pdt);  // [m][K] dt

  const int64_t q0 = (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wv) * m;
  int64_t q = q0 + h;
  if (q >= P.Q) q = -1;
  int64_t node = -1;
  double qt = 0.0;
  bool qvalid = true;
  if (q >= 0) query_load(P, q, node, qt, qvalid);
  const bool bad = q >= 0 && qvalid && node >= P.N;
  if (bad && sl == 0 && P.status != nullptr) atomicAdd(&P.status[TGX_ST_BAD_QUERY_NODE], 1);
  // a padding node (< 0) has an empty window
  const bool live = q >= 0 && qvalid && !bad && node >= 0 && P.has_csr;
  int64_t s0 = 0, s1 = 0;
  if (live) {
    s0 = P.c_off[node];
    s1 = P.c_off[node + 1];
  }

  // ---- the entry at this lane's position if the answer is the window's last K ----
  double t = 0.0;
  int32_t id = -1;
  int64_t eid = -1;
  VT rows[NREG > 0 ? NREG : 1];
#pragma unroll
  for (int k = 0; k < (NREG > 0 ? NREG : 1); ++k) rows[k] = VT{};
  auto load_entry = [&](int64_t x) {
    t = P.c_times[x];
    id = P.c_ids[x];
    if (P.o_eids != nullptr) eid = P.c_eids != nullptr ? P.c_eids[x] : -1;
    if constexpr (NREG > 0) {
      const VT* src = reinterpret_cast<const VT*>(P.c_feats + x * P.row_bytes);
#pragma unroll
      for (int k = 0; k < NREG; ++k)
        if (k < P.nch) rows[k] = src[k];
    }
  };
  bool have = live && sl < K && s1 - K + sl >= s0;
  if (have) load_entry(s1 - K + sl);
  // the search's first round over a window of more than Bp entries, when the query
  // may be inside it (not after the CSR's last time): probe sl at s0 + (sl + 1)
  // step - 1, clamped to the last entry
  const int Bp = 1 << lg;
  const int64_t wlen = s1 - s0;
  const bool probing = live && wlen > Bp && qt <= P.c_tmax;
  const int64_t step = probing ? (wlen + Bp - 1) >> lg : 0;
  double tp = 0.0;
  if (probing) {
    const int64_t pos = s0 + (sl + 1) * step - 1;
    tp = P.c_times[pos < s1 ? pos : s1 - 1];
  }
  // sub-group uniform: lane K - 1 holds entry s1 - 1 whenever the window is not empty
  const double tl = __shfl(t, (h << lg) + K - 1);
  const bool after = !live || s1 == s0 || tl < qt;

  // ---- otherwise: search the window, then load the answer's entries ----
  const uint64_t slow = __ballot(!after);
  if (slow != 0) {  // wave-uniform
    // the lower bound lies in [lo, hi]: after the first round, between the last
    // probe below the query time and the next one
    const uint64_t below = __ballot(probing && tp < qt) >> (h << lg);
    int64_t lo = s0, hi = s1;
    if (probing) {
      const int64_t c = __popcll(Bp == kWave ? below : below & ((uint64_t(1) << Bp) - 1));
      const int64_t nl = s0 + c * step;
      const int64_t pc = s0 + (c + 1) * step - 1;
      lo = nl < s1 ? nl : s1;
      hi = pc < s1 ? pc : s1;
    }
    // every sub-group searches its own query at once (Bp-ary rounds; one query
    // after another with 64-ary rounds took 2 x 3 rounds for C3's hop-2 windows)
    const int64_t cnt = subgroup_lower_bound(P.c_times, lo, hi, qt, !after, sl, h, lg) - s0;
    if (!after) {
      const int take = static_cast<int>(cnt < K ? cnt : K);
      have = sl < K && sl >= K - take;
      if (have) load_entry(s0 + cnt - K + sl);
    }
  }

  // ---- outputs: position sl of query q ----
  const bool out = q >= 0 && sl < K;
  if (P.d_t > 0) {  // launch-uniform
    float dt = 0.0f;
    bool big = false;
    if (out) {
      const double tt = have ? t : 0.0;
      dt = dyg ? static_cast<float>(qt) - static_cast<float>(tt) : static_cast<float>(qt - tt);
      big = (!dyg || have) && !(fabsf(dt) < P.te_dt_small);
      pcode[h * K + sl] = have ? 0 : -1;
      pdt[h * K + sl] = dt;
    }
    const bool te_big = __ballot(big) != 0;
    wave_sync();
    // the wave's valid queries are consecutive from q0
    const int64_t nv = q0 < P.Q ? (P.Q - q0 < m ? P.Q - q0 : m) : 0;
    const int np = static_cast<int>(nv) * K;
    if (np > 0) {
      if (te_big)
        encode_rows<true, false>(P, q0 * K, np, pcode, pdt, s_w, s_b, lane, kWave);
      else
        encode_rows<false, false>(P, q0 * K, np, pcode, pdt, s_w, s_b, lane, kWave);
    }
  }
  if (out) {
    const int64_t o = q * K + sl;
    if constexpr (NREG > 0) {
      VT* dst = reinterpret_cast<VT*>(P.o_feats + o * P.row_bytes);
#pragma unroll
      for (int k = 0; k < NREG; ++k)
        if (k < P.nch) put<false>(dst + k, have ? rows[k] : VT{});
    }
    P.o_ids[o] = have ? id : -1;
    P.o_times[o] = have ? t : 0.0;
    P.o_mask[o] = have ? 1 : 0;
    if (P.o_eids != nullptr) P.o_eids[o] = have ? eid : -1;
  }
}

// Ring-less tiled gather over a frozen CSR whose queries may be split over
// several waves and whose rows go through memory (any width): the launches
// csr_window does not take (fewer queries, rows above 64 bytes, K above 64),
// such as DataPipeline.prepare of 200-event batches on the Engine's frozen CSR.
// Two layouts of a query's `split` waves: at K <= 64 each wave holds all K
// answer entries (lane p: position p) and writes every split-th 64-chunk run of
// the query's rows and encodings; with RANGES (K above 64) the waves own
// consecutive ranges of per = ceil(K / split) <= 64 positions (lane l of wave
// part: position part * per + l) and write those positions' outputs.  (At the
// Engine's K = 32 and 64 the interleaved runs measured 14% faster than ranges;
// at K = 512 only ranges keep one entry per lane.)  With the offsets in, a wave
// loads the entries the window's last K would put at its lanes' positions, the
// window's last time and the first kCopyDepth chunks per lane of its share of
// their rows; when the query comes after its whole window those are the answer
// (query, offsets, entries and first row chunks: three dependent round trips
// before the first store, against five in recent_fused's ring-less copy).
// Otherwise the wave searches the window and reloads.
template <int VEC, bool RANGES>
__global__ __launch_bounds__(kMaxWaves * kWave) void csr_split(Params P) {
  using VT = typename Vec<VEC>::T;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int K = P.K;
  const int split = P.split;
  // the query's waves: `split` of one workgroup, or spread over wg_parts workgroups
  const int wpw = static_cast<int>(blockDim.x) / kWave;
  const int qs = P.wg_parts > 1 ? 0 : wv / split;
  const int part = P.wg_parts > 1 ? static_cast<int>(blockIdx.x % static_cast<unsigned>(P.wg_parts)) * wpw + wv
                                  : wv - qs * split;
  const int per = RANGES ? (K + split - 1) / split : K;
  const int p0 = RANGES ? part * per : 0;
  const int np = K - p0 < per ? (K - p0 > 0 ? K - p0 : 0) : per;  // the wave's positions
  const int pos = p0 + lane;                                      // lane < np
  // the wave's share of the chunks of its positions' rows (and of their
  // encodings): 64-chunk runs from off, every cstride chunks
  const int off = RANGES ? 0 : part * kWave;
  const int cstride = RANGES ? kWave : split * kWave;
  const bool dyg = P.dt_mode == TGX_DT_DYGFORMER;

  float* s_w = reinterpret_cast<float*>(smem);
  float* s_b = s_w + (P.te_bytes / 8);
  if (P.d_t > 0) {  // launch-uniform
    for (int i = threadIdx.x; i < P.d_t; i += blockDim.x) {
      s_w[i] = P.te_w[i];
      s_b[i] = P.te_b != nullptr ? P.te_b[i] : 0.0f;
    }
    __syncthreads();
  }
  uint8_t* wb = smem + P.te_bytes + static_cast<size_t>(wv) * P.wave_bytes;
  int32_t* pcode = reinterpret_cast<int32_t*>(wb);        // [per] 0 entry, -1 pad
  float* pdt = reinterpret_cast<float*>(wb + P.off_pdt);  // [per] dt

  int64_t q = P.wg_parts > 1 ? static_cast<int64_t>(blockIdx.x / static_cast<unsigned>(P.wg_parts))
                              : static_cast<int64_t>(blockIdx.x) * (wpw / split) + qs;
  if (q >= P.Q) q = -1;
  int64_t node = -1;
  double qt = 0.0;
  bool qvalid = true;
  if (q >= 0) query_load(P, q, node, qt, qvalid);
  const bool bad = q >= 0 && qvalid && node >= P.N;
  if (bad && lane == 0 && part == 0 && P.status != nullptr) atomicAdd(&P.status[TGX_ST_BAD_QUERY_NODE], 1);
  // wave-uniform; a padding node (< 0) has an empty window
  const bool live = q >= 0 && qvalid && !bad && node >= 0 && P.has_csr;
  int64_t s0 = 0, s1 = 0;
  if (live) {
    s0 = P.c_off[node];
    s1 = P.c_off[node + 1];
  }

  // ---- if the answer is the window's last K: this lane's entry, the window's last
  // time and the first row chunks of the wave's positions ----
  double t = 0.0, tl = 0.0;
  int32_t id = -1;
  int64_t eid = -1;
  auto load_entry = [&](int64_t x) {
    t = P.c_times[x];
    id = P.c_ids[x];
    if (P.o_eids != nullptr) eid = P.c_eids != nullptr ? P.c_eids[x] : -1;
  };
  bool have = live && lane < np && s1 - K + pos >= s0;
  if (have) load_entry(s1 - K + pos);
  // with ranges only the last wave holds position K - 1
  if (RANGES && live && s1 > s0) tl = P.c_times[s1 - 1];
  const bool fe = P.o_feats != nullptr && P.row_bytes > 0;
  const int nch = P.nch;
  const int total = np * nch;  // chunks of the wave's positions
  const FastDiv dv(nch, P.fd_c);
  const VT* crow = reinterpret_cast<const VT*>(P.c_feats);
  VT v[kCopyDepth];
#pragma unroll
  for (int u = 0; u < kCopyDepth; ++u) {
    const int idx = off + u * cstride + lane;
    v[u] = VT{};
    if (fe && live && idx < total) {
      const int pl = static_cast<int>(dv.div(idx));
      const int64_t x = s1 - K + p0 + pl;
      if (x >= s0) v[u] = crow[x * nch + (idx - pl * nch)];
    }
  }
  if (!RANGES) tl = __shfl(t, K - 1);  // entry s1 - 1 whenever the window is not empty
  const bool after = !live || s1 == s0 || tl < qt;
  // position p >= K - take holds entry base + p
  int64_t base = s1 - K;
  int take = live ? static_cast<int>(s1 - s0 < K ? s1 - s0 : K) : 0;
  if (!after) {  // wave-uniform
    const int64_t cnt = wave_lower_bound<true>(P.c_times, s0, s1, qt, lane) - s0;
    take = static_cast<int>(cnt < K ? cnt : K);
    base = s0 + cnt - K;
    have = lane < np && pos >= K - take;
    if (have) load_entry(base + pos);
  }

  if (q >= 0 && np > 0) {  // wave-uniform
    // ---- feature rows of the wave's positions ----
    if (fe) {
      VT* of = reinterpret_cast<VT*>(P.o_feats) + (q * K + p0) * nch;
      for (int idx0 = off; idx0 < total; idx0 += kCopyDepth * cstride) {
        if (idx0 != off || !after) {
#pragma unroll
          for (int u = 0; u < kCopyDepth; ++u) {
            const int idx = idx0 + u * cstride + lane;
            v[u] = VT{};
            if (idx < total) {
              const int pl = static_cast<int>(dv.div(idx));
              if (p0 + pl >= K - take) v[u] = crow[(base + p0 + pl) * nch + (idx - pl * nch)];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kCopyDepth; ++u) {
          const int idx = idx0 + u * cstride + lane;
          if (idx < total) put<true>(of + idx, v[u]);
        }
      }
    }
    // ---- time encodings of the wave's positions ----
    if (P.d_t > 0) {
      bool big = false;
      if (lane < np) {
        const double tt = have ? t : 0.0;
        const float dt = dyg ? static_cast<float>(qt) - static_cast<float>(tt) : static_cast<float>(qt - tt);
        big = (!dyg || have) && !(fabsf(dt) < P.te_dt_small);
        pcode[lane] = have ? 0 : -1;
        pdt[lane] = dt;
      }
      const bool te_big = __ballot(big) != 0;
      wave_sync();
      // nontemporal encodings beside rows that stream; ordinary stores beside small
      // rows, where the encodings are the launch's bytes (LastFM's 8-byte rows at
      // K = 512: 29.9 -> 25.1 us; with 688-byte rows nontemporal stays faster)
      if (P.te_nt) {
        if (te_big)
          encode_rows<true, true>(P, q * K + p0, np, pcode, pdt, s_w, s_b, off + lane, cstride);
        else
          encode_rows<false, true>(P, q * K + p0, np, pcode, pdt, s_w, s_b, off + lane, cstride);
      } else {
        if (te_big)
          encode_rows<true, false>(P, q * K + p0, np, pcode, pdt, s_w, s_b, off + lane, cstride);
        else
          encode_rows<false, false>(P, q * K + p0, np, pcode, pdt, s_w, s_b, off + lane, cstride);
      }
    }
    // ---- ids / times / mask / edge ids (without ranges: the query's first wave) ----
    if (lane < np && (RANGES || part == 0)) {
      const int64_t o = q * K + pos;
      P.o_ids[o] = have ? id : -1;
      P.o_times[o] = have ? t : 0.0;
      P.o_mask[o] = have ? 1 : 0;
      if (P.o_eids != nullptr) P.o_eids[o] = have ? eid : -1;
    }
  }
}

// stand-alone co-occurrence (FREQ) over id rows: one wavefront per pair.  A
// position is valid by its mask byte, or without masks when its id is not -1;
// counts cover valid positions only (an id of -2^31 marks an invalid one in LDS:
// valid ids are compared only against valid ids)
__global__ __launch_bounds__(64) void co_occurrence_rows(const int32_t* __restrict__ a_ids,
                                                         const int32_t* __restrict__ c_ids,
                                                         const uint8_t* __restrict__ a_mask,
                                                         const uint8_t* __restrict__ c_mask,
                                                         int64_t pairs, int K,
                                                         int32_t* __restrict__ a_cnt,
                                                         int32_t* __restrict__ c_cnt,
                                                         float* __restrict__ pair_count) {
  extern __shared__ int32_t rows[];
  int32_t* A = rows;             // [K] ids
  int32_t* Cc = rows + K;        // [K] ids
  int32_t* Av = rows + 2 * K;    // [K] validity
  int32_t* Cv = rows + 3 * K;
  const int64_t g = blockIdx.x;
  const int lane = threadIdx.x;
  for (int i = lane; i < K; i += kWave) {
    const int32_t x = a_ids[g * K + i];
    const int32_t y = c_ids[g * K + i];
    A[i] = x;
    Cc[i] = y;
    Av[i] = a_mask != nullptr ? (a_mask[g * K + i] != 0) : (x != -1);
    Cv[i] = c_mask != nullptr ? (c_mask[g * K + i] != 0) : (y != -1);
  }
  __syncthreads();
  int pc = 0;
  for (int i0 = 0; i0 < K; i0 += kWave) {
    const int i = i0 + lane;
    int aa = 0, ac = 0, ca = 0, cc = 0;
    bool xv = false;
    if (i < K) {
      const int32_t x = A[i], y = Cc[i];
      xv = Av[i] != 0;
      const bool yv = Cv[i] != 0;
      for (int j = 0; j < K; ++j) {
        const int32_t aj = A[j], cj = Cc[j];
        const bool ajv = Av[j] != 0, cjv = Cv[j] != 0;
        aa += ajv && aj == x;
        ac += cjv && cj == x;
        ca += ajv && aj == y;
        cc += cjv && cj == y;
      }
      if (!xv) aa = ac = 0;
      if (!yv) ca = cc = 0;
      a_cnt[(g * K + i) * 2 + 0] = aa;
      a_cnt[(g * K + i) * 2 + 1] = ac;
      c_cnt[(g * K + i) * 2 + 0] = ca;
      c_cnt[(g * K + i) * 2 + 1] = cc;
    }
    pc += __popcll(__ballot(i < K && xv && ac > 0));
  }
  if (lane == 0 && pair_count != nullptr) pair_count[g] = static_cast<float>(pc);
}

int round16(int x) { return (x + 15) & ~15; }

}  // namespace
}  // namespace tgx

using namespace tgx;

namespace tgx {
namespace {

// Launch configuration of one tgx_recent call: kernel parameters, grid and the
// fused plan (see tgx_recent_launch_shape for the reported fields).
struct Launch {
  Params P;
  PlanParams pl;
  bool want_plan = false;
  bool fuse_plan = false;
  bool empty = false;  // no queries: only the plan (if any) runs
  int64_t blocks = 0;
  int threads = 0;
  size_t lds = 0;
  int qslots = 0;
  int vec = 2;
  int nreg = 0;
  bool noring = false;
  bool window = false;  // csr_window runs the launch
  bool csr_split = false;  // csr_split runs it
  bool csr_ranges = false;  // in position ranges (K above 64)
};

// |dt| below which every encoding argument fl32(fl32(dt w) + b) stays below
// kRevArg for weights |w| <= bw and biases |b| <= bb, rounded down; 0 when the
// bounds are unknown (bw <= 0 or not finite), so that every element takes the
// full-range reduction.  Each of the two float roundings grows a value by at
// most 2^-24 relative; the margin r covers both.
float te_small_dt(float bw, float bb) {
  if (!(bw > 0.0f) || !std::isfinite(bw) || !(bb >= 0.0f) || !std::isfinite(bb)) return 0.0f;
  const double r = 1.0 + std::ldexp(1.0, -22);
  const double lim = static_cast<double>(kRevArg) / r - static_cast<double>(bb);
  if (!(lim > 0.0)) return 0.0f;
  const double t = lim / (static_cast<double>(bw) * r);
  const float f = static_cast<float>(t);
  return static_cast<double>(f) > t ? std::nextafter(f, 0.0f) : f;
}

int setup_recent(const tgx_ring* ring, const tgx_csr* csr, const tgx_recent_args* a, Launch& L) {
  L = Launch{};
  Params& P = L.P;
  P = Params{};
  if (a == nullptr) return fail(TGX_ERR_ARG, "tgx_recent: args is NULL");
  if (a->num_queries < 0 || a->num_groups < 0)
    return fail(TGX_ERR_ARG, "tgx_recent: negative query/group count");
  if (a->k < 1 || a->k > TGX_MAX_K)
    return fail(TGX_ERR_LIMIT, "tgx_recent: k=%d outside [1, %d]", a->k, TGX_MAX_K);
  if (a->group < 1 || a->group > TGX_MAX_GROUP)
    return fail(TGX_ERR_LIMIT, "tgx_recent: group=%d outside [1, %d]", a->group, TGX_MAX_GROUP);
  if (a->num_groups >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "tgx_recent: too many groups");
  const int mode = a->plan != nullptr ? TGX_PLAN_LIST : a->plan_mode;
  if (mode != TGX_PLAN_TILES && mode != TGX_PLAN_EVENTS && mode != TGX_PLAN_LIST)
    return fail(TGX_ERR_ARG, "tgx_recent: unknown plan_mode %d", a->plan_mode);
  if (mode == TGX_PLAN_LIST && a->plan == nullptr)
    return fail(TGX_ERR_ARG, "tgx_recent: TGX_PLAN_LIST needs a plan array");
  // the caller's next ring batch, planned in this launch (or on its own)
  L.want_plan = a->append_b != 0;
  if (L.want_plan) {
    if (ring == nullptr) return fail(TGX_ERR_ARG, "tgx_recent: an append plan needs the ring");
    const int rc = plan_setup("tgx_recent", ring, a->append_src, a->append_dst, a->append_time,
                              a->append_b, a->append_workspace, a->append_workspace_bytes, L.pl);
    if (rc != TGX_OK) return rc;
  }
  const int64_t ngroups_eff = mode == TGX_PLAN_LIST ? a->num_groups : 1;  // events: their tail may hold queries
  if (a->num_queries == 0 || ngroups_eff == 0) {
    L.empty = true;
    return TGX_OK;
  }
  if (a->num_query_groups < 0 || a->num_query_groups > TGX_MAX_QUERY_GROUPS)
    return fail(TGX_ERR_LIMIT, "tgx_recent: %d query groups outside [0, %d]", a->num_query_groups,
                TGX_MAX_QUERY_GROUPS);
  if ((a->num_query_groups == 0 && (a->nodes == nullptr || a->times == nullptr)) ||
      a->out_ids == nullptr || a->out_times == nullptr || a->out_mask == nullptr)
    return fail(TGX_ERR_ARG, "tgx_recent: nodes/times/out_ids/out_times/out_mask must not be NULL");

  int feat_dim = -1, dtype = -1;
  if (ring != nullptr) {
    if (ring->slots < 1 || ring->slots > TGX_MAX_SLOTS)
      return fail(TGX_ERR_LIMIT, "tgx_recent: ring slots=%d outside [1, %d]", ring->slots,
                  TGX_MAX_SLOTS);
    if (ring->ids == nullptr || ring->times == nullptr)
      return fail(TGX_ERR_ARG, "tgx_recent: ring ids/times are NULL");
    P.N = ring->num_nodes;
    P.B = ring->slots;
    P.r_ids = ring->ids;
    P.r_times = ring->times;
    P.r_feats = static_cast<const uint8_t*>(ring->feats);
    P.r_eids = ring->eids;
    P.r_wp = ring->write_pos;
    P.b_pow2 = (P.B & (P.B - 1)) == 0 ? 1 : 0;
    feat_dim = ring->feat_dim;
    dtype = ring->feat_dtype;
  }
  if (csr != nullptr) {
    if (csr->offsets == nullptr || (csr->num_entries > 0 && (csr->ids == nullptr || csr->times == nullptr)))
      return fail(TGX_ERR_ARG, "tgx_recent: csr arrays are NULL");
    if (ring != nullptr && (csr->num_nodes != ring->num_nodes || csr->feat_dim != feat_dim ||
                            csr->feat_dtype != dtype))
      return fail(TGX_ERR_ARG, "tgx_recent: ring and csr disagree on nodes/feat_dim/dtype");
    P.N = csr->num_nodes;
    P.has_csr = csr->num_entries > 0 ? 1 : 0;
    P.c_tmax = csr->max_time;
    P.c_off = csr->offsets;
    P.c_ids = csr->ids;
    P.c_times = csr->times;
    P.c_feats = static_cast<const uint8_t*>(csr->feats);
    P.c_eids = csr->eids;
    feat_dim = csr->feat_dim;
    dtype = csr->feat_dtype;
  }
  if (ring == nullptr && csr == nullptr) {
    // every query is padding; the rows' width comes from a ring or a CSR
    if (a->out_feats != nullptr)
      return fail(TGX_ERR_ARG, "tgx_recent: out_feats needs a ring or a CSR (their feat_dim sizes the rows)");
    P.N = INT64_MAX;
    feat_dim = 0;
    dtype = TGX_F32;
  }
  const int esz = feat_elem_bytes(dtype);
  if (esz == 0) return fail(TGX_ERR_DTYPE, "tgx_recent: unsupported feat dtype %d", dtype);
  if (feat_dim < 0) return fail(TGX_ERR_ARG, "tgx_recent: negative feat_dim");
  P.row_bytes = static_cast<int64_t>(feat_dim) * esz;
  if (a->out_feats != nullptr && P.row_bytes > 0) {
    if ((ring != nullptr && ring->feats == nullptr) || (P.has_csr && csr->feats == nullptr))
      return fail(TGX_ERR_ARG, "tgx_recent: feature arrays are NULL");
  }
  P.nodes = a->nodes;
  P.qtimes = a->times;
  P.ngroups = a->num_query_groups;
  {
    int64_t off = 0;
    int per_event = 0;
    const int ev_groups = a->event_query_groups > 0 ? a->event_query_groups : a->num_query_groups;
    if (mode == TGX_PLAN_EVENTS && (a->event_query_groups < 0 || ev_groups > a->num_query_groups))
      return fail(TGX_ERR_ARG, "tgx_recent: event_query_groups=%d outside [0, %d]", a->event_query_groups,
                  a->num_query_groups);
    for (int g = 0; g < a->num_query_groups; ++g) {
      const tgx_query_group& qg = a->query_groups[g];
      if (qg.count < 0 || qg.times_per < 1 || (qg.count > 0 && (qg.nodes == nullptr || qg.times == nullptr)) ||
          (qg.flags & ~TGX_QG_NODES_I32) != 0)
        return fail(TGX_ERR_ARG, "tgx_recent: bad query group %d", g);
      P.gn[g] = qg.nodes;
      P.gv[g] = qg.valid;
      P.gi32[g] = (qg.flags & TGX_QG_NODES_I32) != 0;
      P.gt[g] = qg.times;
      P.gdiv[g] = qg.times_per;
      P.goff[g] = off;
      off += qg.count;
      if (mode == TGX_PLAN_EVENTS && g >= ev_groups) continue;  // a tail group
      per_event += qg.times_per;
      if (mode == TGX_PLAN_EVENTS && qg.count != a->num_groups * qg.times_per)
        return fail(TGX_ERR_ARG, "tgx_recent: event-major plan: query group %d holds %lld queries, "
                    "not num_groups x times_per = %lld", g, (long long)qg.count,
                    (long long)(a->num_groups * qg.times_per));
    }
    for (int g = a->num_query_groups; g <= TGX_MAX_QUERY_GROUPS; ++g) P.goff[g] = off;
    if (a->num_query_groups > 0 && off != a->num_queries)
      return fail(TGX_ERR_ARG, "tgx_recent: query groups hold %lld queries, num_queries is %lld",
                  (long long)off, (long long)a->num_queries);
    if (mode == TGX_PLAN_EVENTS && (a->num_query_groups == 0 || per_event != a->group))
      return fail(TGX_ERR_ARG, "tgx_recent: event-major plan needs query groups whose times_per "
                  "sum to group (%d)", a->group);
    if (mode == TGX_PLAN_EVENTS) {
      // every query group holds exactly num_groups x times_per queries (checked
      // above), so slot j of event g < num_groups is always a query
      int j = 0, before = 0;
      P.ev_code[0] = P.ev_code[1] = 0;
      P.ev_b = a->num_groups;
      P.ev_tail = P.goff[ev_groups];
      for (int g = 0; g < ev_groups; ++g) {
        const int per = a->query_groups[g].times_per;
        for (int i = 0; i < per; ++i, ++j) {
          const uint64_t c = static_cast<uint64_t>(before | (per << 4) | (i << 8));
          P.ev_code[j < 5 ? 0 : 1] |= c << (12 * (j < 5 ? j : j - 5));
        }
        before += per;
      }
    }
  }
  if (mode == TGX_PLAN_LIST) P.ev_b = a->num_groups;  // pairs: every group of the list
  P.Q = a->num_queries;
  P.K = a->k;
  P.plan = a->plan;
  P.plan_mode = mode;
  P.G = a->group;
  P.o_ids = a->out_ids;
  P.o_times = a->out_times;
  P.o_feats = static_cast<uint8_t*>(a->out_feats);
  P.o_mask = a->out_mask;
  P.o_eids = a->out_eids;
  P.d_t = a->d_t;
  if (a->d_t < 0 || a->d_t > TGX_MAX_DT)
    return fail(TGX_ERR_LIMIT, "tgx_recent: d_t=%d outside [0, %d]", a->d_t, TGX_MAX_DT);
  if (a->d_t > 0 && (a->te_w == nullptr || a->out_te == nullptr))
    return fail(TGX_ERR_ARG, "tgx_recent: d_t > 0 needs te_w and out_te");
  if (a->dt_mode != TGX_DT_DYGFORMER && a->dt_mode != TGX_DT_TGN)
    return fail(TGX_ERR_ARG, "tgx_recent: unknown dt_mode %d", a->dt_mode);
  P.te_w = a->te_w;
  P.te_b = a->te_b;
  P.te_dt_small = te_small_dt(a->te_bound_w, a->te_bound_b);
  P.dt_mode = a->dt_mode;
  P.o_te = a->out_te;
  P.te_vec4 = (a->d_t % 4 == 0 && aligned16(a->out_te)) ? 1 : 0;
  if (a->co_mode != TGX_CO_NONE && a->co_mode != TGX_CO_FREQ && a->co_mode != TGX_CO_DYGFORMER)
    return fail(TGX_ERR_ARG, "tgx_recent: unknown co_mode %d", a->co_mode);
  if (a->co_mode != TGX_CO_NONE && (a->group < 2 || a->co_a == nullptr || a->co_c == nullptr))
    return fail(TGX_ERR_ARG, "tgx_recent: co-occurrence needs group >= 2 and co_a/co_c");
  if (a->co_mode != TGX_CO_NONE && mode == TGX_PLAN_TILES)
    return fail(TGX_ERR_ARG, "tgx_recent: co-occurrence pairs queries 0 and 1 of a plan group: it "
                "needs TGX_PLAN_EVENTS or a plan array");
  P.co_mode = a->co_mode;
  P.co_a = a->co_a;
  P.co_c = a->co_c;
  P.co_pair = a->co_pair;
  P.status = a->status;

  const int K = a->k;
  // LDS candidates: the CSR window and the ring slots.  A tiled launch without a
  // ring runs csr_window or csr_split (below), which stage no candidates; the
  // split rule sizes it as a recent_fused launch without them
  L.noring = ring == nullptr && mode == TGX_PLAN_TILES;
  P.cand_cap = L.noring ? 0 : (P.has_csr ? K : 0) + P.B;
  auto wave_lds = [&](int m) {
    return round16(m * P.cand_cap * 16) + round16(m * K * 4) * 3 + round16(m * K * 8) *
           (a->out_eids != nullptr ? 2 : 1) + round16(m * 24);
  };
  // Queries per wave.  Packing m = 64 / Bp queries into sub-groups of Bp >= B
  // lanes (Bp at least 16, the wave's LDS within 12 KB) pays off only when the
  // rows ride in registers and the batch has more queries than the device has
  // wave slots (one round of waves instead of two); otherwise, and with plan
  // groups, one query per wave keeps the most waves in flight.
  const bool small_rows = P.B > 0 && a->out_feats != nullptr && P.row_bytes > 0 &&
                          P.row_bytes <= 64 && P.row_bytes % 16 == 0;
  int lg = 6;
  if (mode == TGX_PLAN_TILES && small_rows && a->num_queries > kPackMinQueries) {
    lg = 4;
    while ((1 << lg) < P.B) ++lg;
    while (lg < 6 && wave_lds(kWave >> lg) > 12 * 1024) ++lg;
  }
  P.m = kWave >> lg;
  P.lg_bp = lg;
  P.te_bytes = 2 * round16(a->d_t * 4);
  P.off_cid = round16(P.m * P.cand_cap * 8);
  P.off_code = P.off_cid + round16(P.m * P.cand_cap * 4);
  P.off_pcode = P.off_code + round16(P.m * P.cand_cap * 4);
  P.off_pdt = P.off_pcode + round16(P.m * K * 4);
  P.off_pid = P.off_pdt + round16(P.m * K * 4);
  P.off_pt = P.off_pid + round16(P.m * K * 4);
  P.off_pe = P.off_pt + round16(P.m * K * 8);
  P.off_tab = P.off_pe + (a->out_eids != nullptr ? round16(P.m * K * 8) : 0);  // edge ids only when asked
  P.wave_bytes = P.off_tab + round16(P.m * 24);
  // split: with one query per wave, up to 8 waves share each query's outputs while
  // the launch stays within kSplitMaxWaves waves; and up to 8 while each wave's share of a
  // query's output bytes stays at least kSplitBytes, so a grid of long copies
  // (large rows, large K) ends with a shorter tail of lone waves.  A workgroup
  // holds at most kMaxWaves waves (the kernel's launch bound): its query slots
  // (the plan group, or `group` consecutive tiles) times split.
  const int qwant = mode != TGX_PLAN_TILES ? a->group : 1;
  // waves whose LDS fits the CU's 160 KB next to the encoder weights (a large K
  // with a CSR window takes about 24 KB per wave)
  const int lds_waves = static_cast<int>((160 * 1024 - P.te_bytes) / P.wave_bytes);
  const int wave_cap = lds_waves < kMaxWaves ? lds_waves : kMaxWaves;
  // A launch whose workgroups all fit on the device at once at one wave per
  // query, with the LDS bounding the workgroups per CU (a large K), splits only
  // while they still do: a split that leaves workgroups for a second round is
  // slower than fewer waves per query (LastFM's shape, 600 queries at K = 512:
  // 4 waves each made one 91 KB workgroup per CU and three rounds)
  auto fits = [&](int sp) {
    const int64_t wg_bytes = static_cast<int64_t>(P.te_bytes) + static_cast<int64_t>(qwant) * sp * P.wave_bytes;
    const int64_t per_cu = (160 * 1024) / wg_bytes;
    const int64_t groups = mode == TGX_PLAN_TILES ? a->num_queries : (a->num_queries + qwant - 1) / qwant;
    return per_cu >= kMaxWaves || groups <= kDeviceCUs * per_cu;
  };
  const bool one_round = fits(1);
  auto resident = [&](int sp) { return !one_round || fits(sp); };
  int split = 1;
  if (P.m == 1) {
    while (split < 8 && a->num_queries * (split * 2) <= kSplitMaxWaves && qwant * split * 2 <= wave_cap &&
           resident(split * 2))
      split *= 2;
    const int64_t qbytes = static_cast<int64_t>(K) * (P.row_bytes + 4 * a->d_t + 13);
    while (split < 8 && qbytes / (split * 2) >= kSplitBytes && qwant * split * 2 <= wave_cap &&
           resident(split * 2))
      split *= 2;
  }
  const int lg_split = split == 1 ? 0 : split == 2 ? 1 : split == 4 ? 2 : 3;  // split is 1, 2, 4 or 8
  P.split = mode == TGX_PLAN_TILES ? split : lg_split;
  // tiles: `group` query slots per workgroup; a query split over several waves
  // takes a workgroup of its own (so a small launch spreads over more CUs: C1's
  // 600 queries, 4 waves each, ran 0.5 us faster in 600 workgroups than in 300)
  int qslots = a->group;
  if (mode == TGX_PLAN_TILES && split > 1) qslots = 1;
  if (mode == TGX_PLAN_TILES && qslots * split > wave_cap) qslots = wave_cap > split ? wave_cap / split : 1;
  int waves = qslots * split;
  if (waves < 1 || waves > kMaxWaves)
    return fail(TGX_ERR_LIMIT, "tgx_recent: %d wavefronts per workgroup outside [1, %d]", waves, kMaxWaves);
  int64_t nblocks = a->num_groups;
  if (mode == TGX_PLAN_EVENTS) nblocks += (a->num_queries - P.ev_tail + a->group - 1) / a->group;
  if (mode == TGX_PLAN_TILES) {
    const int64_t ntiles = (a->num_queries + P.m - 1) / P.m;
    nblocks = (ntiles + qslots - 1) / qslots;
  }
  size_t lds = static_cast<size_t>(P.te_bytes) + static_cast<size_t>(waves) * P.wave_bytes;
  if (lds > 160 * 1024) return fail(TGX_ERR_LIMIT, "tgx_recent: %zu bytes of LDS needed", lds);

  int vec = 2;
  const bool fe = a->out_feats != nullptr && P.row_bytes > 0;
  auto al = [](const void* p, unsigned m) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & m) == 0; };
  if (P.row_bytes % 16 == 0 && (!fe || (al(P.r_feats, 15) && al(P.c_feats, 15) && al(P.o_feats, 15))))
    vec = 16;
  else if (P.row_bytes % 4 == 0 && (!fe || (al(P.r_feats, 3) && al(P.c_feats, 3) && al(P.o_feats, 3))))
    vec = 4;
  P.nch = static_cast<int>(P.row_bytes / vec);
  // FastDiv(n) is exact for x * n < 2^32; its largest dividends: K * nch
  // feature chunks (divided by nch), m*K*d_t encodings (by d_t or d_t / 4) and
  // m*K positions (by K)
  if (static_cast<uint64_t>(K) * static_cast<uint64_t>(P.nch) * static_cast<uint64_t>(P.nch) >=
      (uint64_t(1) << 32))
    return fail(TGX_ERR_LIMIT, "tgx_recent: k=%d with %lld-byte rows (%d chunks of %d bytes) exceeds "
                "the kernel's index range", K, (long long)P.row_bytes, P.nch, vec);
  P.fd_k = FastDiv::magic(static_cast<uint32_t>(P.K));
  P.fd_q = FastDiv::magic(static_cast<uint32_t>(P.d_t / 4));
  P.fd_d = FastDiv::magic(static_cast<uint32_t>(P.d_t));
  P.fd_c = FastDiv::magic(static_cast<uint32_t>(P.nch));
  // rows of at most 4 16-byte chunks ride in registers with the ring slot
  int nreg = 0;
  if (vec == 16 && fe && P.B > 0) nreg = P.nch <= 2 ? 2 : (P.nch <= 4 ? 4 : 0);
  // A ring-less tiled launch at K <= 64 whose queries take one wave each, with
  // rows of at most 4 16-byte chunks (or none), runs csr_window instead: m =
  // 64 / Bp queries per wave in sub-groups of Bp >= max(K, 16) lanes, `group`
  // waves per workgroup
  L.window = L.noring && K <= kWave && split == 1 && (!fe || (vec == 16 && P.nch <= 4));
  if (L.window) {
    int lgw = 4;
    while ((1 << lgw) < K) ++lgw;
    P.lg_bp = lgw;
    P.m = kWave >> lgw;
    P.off_pdt = round16(P.m * K * 4);
    P.wave_bytes = 2 * round16(P.m * K * 4);
    qslots = a->group;
    waves = qslots;
    const int64_t nwaves = (a->num_queries + P.m - 1) / P.m;
    nblocks = (nwaves + qslots - 1) / qslots;
    lds = static_cast<size_t>(P.te_bytes) + static_cast<size_t>(waves) * P.wave_bytes;
    nreg = fe ? (P.nch <= 2 ? 2 : 4) : 0;
  }
  // the other ring-less tiled launches (split queries, rows through memory, K
  // above 64) run csr_split: recent_fused's split; above K = 64 in position
  // ranges, the split raised to a power of two >= K / 64 (each wave owns at most 64
  // positions; its LDS is two words per position, so the split never leaves
  // workgroups for a second round)
  L.csr_split = L.noring && !L.window;
  L.csr_ranges = K > kWave;
  if (L.csr_split) {
    int sp = split;
    while (sp * kWave < K) sp *= 2;  // K <= TGX_MAX_K = 8 x 64
    if (sp != split) {
      split = sp;
      P.split = split;
      qslots = 1;
      waves = split;
      nblocks = a->num_queries;
    }
    // LDS: pcode and dt of the wave's positions (all K without ranges)
    const int per = L.csr_ranges ? (K + split - 1) / split : K;
    P.off_pdt = round16(per * 4);
    P.wave_bytes = 2 * round16(per * 4);
    // a query's waves spread over workgroups of kSplitGroupWaves (its waves share
    // nothing but the encoder weights, which each workgroup loads): finer
    // workgroups even out the CUs
    if (qslots == 1 && split > kSplitGroupWaves) {
      P.wg_parts = split / kSplitGroupWaves;
      waves = kSplitGroupWaves;
      nblocks = a->num_queries * P.wg_parts;
    }
    lds = static_cast<size_t>(P.te_bytes) + static_cast<size_t>(waves) * P.wave_bytes;
    P.te_nt = P.row_bytes >= kNtRowBytes ? 1 : 0;
  }

  // fused plan: one plan workgroup per blockDim entries, dispatched first
  L.fuse_plan = L.want_plan && plan_fused_ok(L.pl);
  P.pl = L.pl;
  P.plan_blocks = L.fuse_plan ? static_cast<int>((L.pl.n + kWave * waves - 1) / (kWave * waves)) : 0;
  L.lds = L.fuse_plan ? std::max(lds, plan_lds_bytes(kWave * waves)) : lds;
  L.blocks = nblocks + P.plan_blocks;
  if (L.blocks >= (int64_t(1) << 31)) return fail(TGX_ERR_LIMIT, "tgx_recent: grid too large");
  L.threads = kWave * waves;
  L.qslots = qslots;
  L.vec = vec;
  L.nreg = nreg;
  return TGX_OK;
}

}  // namespace
}  // namespace tgx

extern "C" int tgx_recent(const tgx_ring* ring, const tgx_csr* csr, const tgx_recent_args* a,
                          void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  Launch L;
  int rc = setup_recent(ring, csr, a, L);
  if (rc != TGX_OK) return rc;
  if (L.empty) return L.want_plan ? launch_plan(L.pl, stream) : TGX_OK;
  hipEvent_t ev0 = static_cast<hipEvent_t>(a->timing_start);
  hipEvent_t ev1 = static_cast<hipEvent_t>(a->timing_stop);
  if ((ev0 == nullptr) != (ev1 == nullptr))
    return fail(TGX_ERR_ARG, "tgx_recent: timing_start and timing_stop must both be set or both NULL");
  static std::once_flag attr_once;
  std::call_once(attr_once, [] {
    const void* fns[] = {reinterpret_cast<const void*>(recent_fused<16, 0, false>),
                         reinterpret_cast<const void*>(recent_fused<16, 2, false>),
                         reinterpret_cast<const void*>(recent_fused<16, 4, false>),
                         reinterpret_cast<const void*>(recent_fused<4, 0, false>),
                         reinterpret_cast<const void*>(recent_fused<2, 0, false>),
                         reinterpret_cast<const void*>(recent_fused<16, 0, true>),
                         reinterpret_cast<const void*>(recent_fused<16, 2, true>),
                         reinterpret_cast<const void*>(recent_fused<16, 4, true>),
                         reinterpret_cast<const void*>(recent_fused<4, 0, true>),
                         reinterpret_cast<const void*>(recent_fused<2, 0, true>)};
    for (const void* f : fns)
      (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipGetLastError();
  });
  const dim3 grid(static_cast<unsigned>(L.blocks));
  const dim3 block(static_cast<unsigned>(L.threads));
  auto launch = [&](auto kernel) {
    if (ev0 != nullptr)
      hipExtLaunchKernelGGL(kernel, grid, block, L.lds, stream, ev0, ev1, 0, L.P);
    else
      hipLaunchKernelGGL(kernel, grid, block, L.lds, stream, L.P);
  };
  // a tiled launch runs the kernel's TILES copy
  const bool tiles = L.P.plan_mode == TGX_PLAN_TILES;
  auto pick = [&](auto k_tiles, auto k_other) {
    if (tiles)
      launch(k_tiles);
    else
      launch(k_other);
  };
  if (L.window) {
    if (L.nreg == 2)
      launch(csr_window<2>);
    else if (L.nreg == 4)
      launch(csr_window<4>);
    else
      launch(csr_window<0>);
  } else if (L.csr_split) {
    if (L.csr_ranges) {
      if (L.vec == 16)
        launch(csr_split<16, true>);
      else if (L.vec == 4)
        launch(csr_split<4, true>);
      else
        launch(csr_split<2, true>);
    } else {
      if (L.vec == 16)
        launch(csr_split<16, false>);
      else if (L.vec == 4)
        launch(csr_split<4, false>);
      else
        launch(csr_split<2, false>);
    }
  } else if (L.vec == 16) {
    if (L.nreg == 2)
      pick(recent_fused<16, 2, true>, recent_fused<16, 2, false>);
    else if (L.nreg == 4)
      pick(recent_fused<16, 4, true>, recent_fused<16, 4, false>);
    else
      pick(recent_fused<16, 0, true>, recent_fused<16, 0, false>);
  } else if (L.vec == 4) {
    pick(recent_fused<4, 0, true>, recent_fused<4, 0, false>);
  } else {
    pick(recent_fused<2, 0, true>, recent_fused<2, 0, false>);
  }
  rc = check_launch(L.window ? "csr_window" : L.csr_split ? "csr_split" : "recent_fused");
  if (rc != TGX_OK || !L.want_plan || L.fuse_plan) return rc;
  return launch_plan(L.pl, stream);  // batches beyond the fused plan's size
}

extern "C" int tgx_recent_launch_shape(const tgx_ring* ring, const tgx_csr* csr,
                                       const tgx_recent_args* a, int64_t shape[8]) {
  if (shape == nullptr) return fail(TGX_ERR_ARG, "tgx_recent_launch_shape: shape is NULL");
  for (int i = 0; i < 8; ++i) shape[i] = 0;
  Launch L;
  const int rc = setup_recent(ring, csr, a, L);
  if (rc != TGX_OK || L.empty) return rc;
  shape[0] = L.blocks;
  shape[1] = L.threads;
  shape[2] = static_cast<int64_t>(L.lds);
  shape[3] = L.P.m;
  shape[4] = L.P.plan_mode == TGX_PLAN_TILES ? L.P.split / (L.P.wg_parts > 1 ? L.P.wg_parts : 1)
                                             : 1 << L.P.split;
  shape[5] = static_cast<int64_t>(L.qslots) * L.P.m;
  shape[6] = L.P.plan_blocks;
  shape[7] = L.vec;
  return TGX_OK;
}

extern "C" int tgx_co_occurrence(const int32_t* a_ids, const int32_t* c_ids, const uint8_t* a_mask,
                                 const uint8_t* c_mask, int64_t pairs, int32_t k, int32_t* a_cnt,
                                 int32_t* c_cnt, float* pair_count, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (pairs < 0 || k < 0) return fail(TGX_ERR_ARG, "tgx_co_occurrence: negative size");
  if (k > 4096) return fail(TGX_ERR_LIMIT, "tgx_co_occurrence: k=%d above 4096", k);
  if (pairs >= (int64_t(1) << 31)) return fail(TGX_ERR_LIMIT, "tgx_co_occurrence: too many pairs");
  if (pairs == 0 || k == 0) return TGX_OK;
  if (a_ids == nullptr || c_ids == nullptr || a_cnt == nullptr || c_cnt == nullptr)
    return fail(TGX_ERR_ARG, "tgx_co_occurrence: NULL pointer");
  hipLaunchKernelGGL(co_occurrence_rows, dim3(static_cast<unsigned>(pairs)), dim3(kWave),
                     4 * k * sizeof(int32_t), stream, a_ids, c_ids, a_mask, c_mask, pairs, k, a_cnt,
                     c_cnt, pair_count);
  return check_launch("co_occurrence_rows");
}
