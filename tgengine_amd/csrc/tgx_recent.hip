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
// Mapping.  One wavefront per query: lanes hold the B <= 64 ring slots, a
// counting rank over the wave's LDS candidate list orders them, and the same
// wave then streams the K feature rows (16-byte loads/stores, lanes spread
// over rows*chunks so every access is coalesced) and the K x d_t encodings
// (float4 stores, cosine evaluated in float64 from the exact fp32 argument).
// A workgroup holds `group` queries so a (src, dst) pair meets in one LDS.
#include "tgx_internal.h"
#include <hip/hip_ext.h>
#include "tgx_cos.h"

namespace tgx {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Params {
  // ring
  int64_t N;
  int B;  // 0 when there is no ring
  const int32_t* r_ids;
  const double* r_times;
  const uint8_t* r_feats;
  const int64_t* r_eids;
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
  const int64_t* gn[TGX_MAX_QUERY_GROUPS];
  const double* gt[TGX_MAX_QUERY_GROUPS];
  int64_t goff[TGX_MAX_QUERY_GROUPS + 1];
  int gdiv[TGX_MAX_QUERY_GROUPS];
  int64_t Q;
  int K;
  const int32_t* plan;
  int G;
  // outputs
  int64_t row_bytes;
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
  // LDS layout
  int te_bytes;
  int wave_bytes;
  int cand_cap;
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

// smallest i in [lo, hi] with i == hi or t[i] >= q (t ascending); wave-uniform result
__device__ __forceinline__ int64_t wave_lower_bound(const double* __restrict__ t, int64_t lo,
                                                    int64_t hi, double q, int lane) {
  while (hi - lo > kWave) {
    const int64_t step = (hi - lo + kWave - 1) / kWave;
    const int64_t pos = lo + static_cast<int64_t>(lane + 1) * step - 1;
    const bool pr = pos < hi && t[pos] < q;
    const int c = __popcll(__ballot(pr));
    const int64_t pc = lo + static_cast<int64_t>(c + 1) * step - 1;
    lo = lo + static_cast<int64_t>(c) * step;
    hi = pc < hi ? pc : hi;
  }
  const int64_t pos = lo + lane;
  const bool pr = pos < hi && t[pos] < q;
  return lo + __popcll(__ballot(pr));
}

__device__ __forceinline__ int64_t query_of(const Params& P, int64_t g, int j) {
  if (j >= P.G) return -1;
  const int64_t slot = g * P.G + j;
  int64_t q;
  if (P.plan != nullptr)
    q = P.plan[slot];
  else
    q = slot;
  return (q >= 0 && q < P.Q) ? q : -1;
}

__device__ __forceinline__ void query_load(const Params& P, int64_t q, int64_t& node, double& qt) {
  if (P.ngroups == 0) {
    node = P.nodes[q];
    qt = P.qtimes[q];
    return;
  }
  int g = 0;
  while (g + 1 < P.ngroups && q >= P.goff[g + 1]) ++g;
  const int64_t l = q - P.goff[g];
  node = P.gn[g][l];
  qt = P.gt[g][P.gdiv[g] == 1 ? l : static_cast<int64_t>(static_cast<uint32_t>(l) / static_cast<uint32_t>(P.gdiv[g]))];
}

__device__ __forceinline__ int64_t query_node(const Params& P, int64_t q) {
  int64_t node;
  double qt;
  query_load(P, q, node, qt);
  return node;
}

template <int VEC>
__global__ __launch_bounds__(512) void recent_fused(Params P) {
  using VT = typename Vec<VEC>::T;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int64_t g = blockIdx.x;
  const int K = P.K;
  const int B = P.B;

  float* s_w = reinterpret_cast<float*>(smem);
  float* s_b = s_w + (P.te_bytes / 8);
  for (int i = threadIdx.x; i < P.d_t; i += blockDim.x) {
    s_w[i] = P.te_w[i];
    s_b[i] = P.te_b != nullptr ? P.te_b[i] : 0.0f;
  }
  uint8_t* wbase = smem + P.te_bytes + static_cast<size_t>(wv) * P.wave_bytes;
  const int C = P.cand_cap;
  double* ct = reinterpret_cast<double*>(wbase);
  int32_t* cid = reinterpret_cast<int32_t*>(wbase + C * 8);
  int32_t* ccode = reinterpret_cast<int32_t*>(wbase + C * 12);
  int32_t* pcode = reinterpret_cast<int32_t*>(wbase + C * 16);
  float* pdt = reinterpret_cast<float*>(wbase + C * 16 + K * 4);
  int32_t* pid = reinterpret_cast<int32_t*>(wbase + C * 16 + K * 8);

  const int64_t q = query_of(P, g, wv);
  const bool active = q >= 0;
  int64_t node = -1;
  double qt = 0.0;
  if (active) query_load(P, q, node, qt);
  const bool bad = active && node >= P.N;
  if (bad && lane == 0 && P.status != nullptr) atomicAdd(&P.status[TGX_ST_BAD_QUERY_NODE], 1);
  const int64_t ur = node < 0 ? 0 : node;

  // ---- candidates: CSR window, then valid ring slots (compacted) ----
  int ncand = 0;
  int64_t cbase = 0;
  if (active && !bad && P.has_csr && node >= 0) {
    const int64_t s0 = P.c_off[node];
    const int64_t s1 = P.c_off[node + 1];
    const int64_t cnt = wave_lower_bound(P.c_times, s0, s1, qt, lane) - s0;
    const int take = static_cast<int>(cnt < K ? cnt : K);
    cbase = s0 + cnt - take;
    for (int j = lane; j < take; j += kWave) {
      ct[j] = P.c_times[cbase + j];
      cid[j] = P.c_ids[cbase + j];
      ccode[j] = B + j;
    }
    ncand = take;
  }
  if (active && !bad && B > 0) {
    int32_t rid = -1;
    double rt = 0.0;
    bool v = false;
    if (lane < B) {
      rid = P.r_ids[ur * B + lane];
      rt = P.r_times[ur * B + lane];
      v = (rid != -1) && (rt < qt);
    }
    const uint64_t m = __ballot(v);
    if (v) {
      const int at = ncand + __popcll(m & ((uint64_t(1) << lane) - 1));
      ct[at] = rt;
      cid[at] = rid;
      ccode[at] = lane;
    }
    ncand += __popcll(m);
  }
  __syncthreads();

  // ---- rank: position of each candidate among the V most recent ----
  const int V = ncand < K ? ncand : K;
  const int drop = ncand - V;
  for (int p = lane; p < K - V; p += kWave) pcode[p] = -1;
  for (int c = lane; c < ncand; c += kWave) {
    const double tc = ct[c];
    int r = 0;
    for (int c2 = 0; c2 < ncand; ++c2) {
      const double t2 = ct[c2];
      r += (t2 < tc) || (t2 == tc && c2 < c);
    }
    if (r >= drop) pcode[K - V + (r - drop)] = c;
  }
  __syncthreads();

  // ---- ids / times / mask / edge ids; per-position dt and source code ----
  if (active) {
    for (int p = lane; p < K; p += kWave) {
      const int c = pcode[p];
      int32_t id = -1;
      double t = 0.0;
      uint8_t mk = 0;
      int64_t e = -1;
      int code = -1;
      if (c >= 0) {
        id = cid[c];
        t = ct[c];
        mk = 1;
        code = ccode[c];
        if (P.o_eids != nullptr) {
          if (code < B)
            e = P.r_eids != nullptr ? P.r_eids[ur * B + code] : -1;
          else
            e = P.c_eids != nullptr ? P.c_eids[cbase + (code - B)] : -1;
        }
      }
      const int64_t o = q * K + p;
      P.o_ids[o] = id;
      P.o_times[o] = t;
      P.o_mask[o] = mk;
      if (P.o_eids != nullptr) P.o_eids[o] = e;
      float dt;
      if (P.dt_mode == TGX_DT_DYGFORMER)
        dt = static_cast<float>(qt) - static_cast<float>(t);
      else
        dt = static_cast<float>(qt - t);
      pdt[p] = dt;
      pid[p] = id;
      pcode[p] = code;
    }
  } else {
    for (int p = lane; p < K; p += kWave) {
      pid[p] = -1;
      pcode[p] = -1;
    }
  }
  __syncthreads();

  if (active) {
    // ---- feature rows: K rows x nch chunks of VEC bytes, lane-flattened ----
    if (P.o_feats != nullptr && P.row_bytes > 0) {
      const int nch = static_cast<int>(P.row_bytes / VEC);
      const int64_t total = static_cast<int64_t>(K) * nch;
      const int sp = kWave / nch, sc = kWave % nch;
      int p = lane / nch, c = lane % nch;
      uint8_t* obase = P.o_feats + q * K * P.row_bytes;
      const uint8_t* rbase = B > 0 ? P.r_feats + ur * B * P.row_bytes : nullptr;
      const uint8_t* cbase_f = P.has_csr ? P.c_feats + cbase * P.row_bytes : nullptr;
      for (int64_t idx = lane; idx < total; idx += 4 * kWave) {
        VT v[4];
        VT* dptr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          dptr[u] = nullptr;
          v[u] = VT{};
          if (idx + u * kWave < total) {
            const int code = pcode[p];
            if (code >= 0) {
              const uint8_t* s = code < B ? rbase + static_cast<int64_t>(code) * P.row_bytes
                                          : cbase_f + static_cast<int64_t>(code - B) * P.row_bytes;
              v[u] = reinterpret_cast<const VT*>(s)[c];
            }
            dptr[u] = reinterpret_cast<VT*>(obase + static_cast<int64_t>(p) * P.row_bytes) + c;
          }
          c += sc;
          p += sp;
          if (c >= nch) {
            c -= nch;
            ++p;
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (dptr[u] != nullptr) __builtin_nontemporal_store(v[u], dptr[u]);
      }
    }

    // ---- time encoding: K rows x d_t ----
    if (P.d_t > 0) {
      const bool dyg = P.dt_mode == TGX_DT_DYGFORMER;
      const bool has_b = P.te_b != nullptr;
      float* tbase = P.o_te + q * K * static_cast<int64_t>(P.d_t);
      if (P.te_vec4) {
        const int nq = P.d_t / 4;
        const int total = K * nq;
        const int sp = kWave / nq, sc = kWave % nq;
        int p = lane / nq, c = lane % nq;
        const f32x4* w4 = reinterpret_cast<const f32x4*>(s_w);
        const f32x4* b4 = reinterpret_cast<const f32x4*>(s_b);
        f32x4* out4 = reinterpret_cast<f32x4*>(tbase);
        for (int idx = lane; idx < total; idx += kWave) {
          f32x4 o = {0.f, 0.f, 0.f, 0.f};
          if (!dyg || pcode[p] >= 0) {
            const float dt = pdt[p];
            f32x4 a = dt * w4[c];
            if (has_b) a = a + b4[c];
            const float amax = fmaxf(fmaxf(fabsf(a[0]), fabsf(a[1])), fmaxf(fabsf(a[2]), fabsf(a[3])));
            if (__builtin_expect(amax < kBigArg, 1)) {
              o[0] = cos_fast(a[0]);
              o[1] = cos_fast(a[1]);
              o[2] = cos_fast(a[2]);
              o[3] = cos_fast(a[3]);
            } else {
              o[0] = cos_slow(a[0]);
              o[1] = cos_slow(a[1]);
              o[2] = cos_slow(a[2]);
              o[3] = cos_slow(a[3]);
            }
          }
          __builtin_nontemporal_store(o, out4 + idx);
          c += sc;
          p += sp;
          if (c >= nq) {
            c -= nq;
            ++p;
          }
        }
      } else {
        const int total = K * P.d_t;
        for (int idx = lane; idx < total; idx += kWave) {
          const int p = idx / P.d_t, j = idx - p * P.d_t;
          float o = 0.f;
          if (!dyg || pcode[p] >= 0) {
            float a = pdt[p] * s_w[j];
            if (has_b) a = a + s_b[j];
            o = fabsf(a) < kBigArg ? cos_fast(a) : cos_slow(a);
          }
          tbase[static_cast<int64_t>(p) * P.d_t + j] = o;
        }
      }
    }
  }

  // ---- co-occurrence of the group's (query 0, query 1) pair ----
  if (P.co_mode != TGX_CO_NONE) {
    __syncthreads();
    const int64_t qa = query_of(P, g, 0), qc = query_of(P, g, 1);
    if (qa >= 0 && qc >= 0 && wv < 2) {
      const int32_t* A = reinterpret_cast<const int32_t*>(smem + P.te_bytes + C * 16 + K * 8);
      const int32_t* Cc =
          reinterpret_cast<const int32_t*>(smem + P.te_bytes + P.wave_bytes + C * 16 + K * 8);
      if (P.co_mode == TGX_CO_FREQ) {
        const int32_t* X = wv == 0 ? A : Cc;
        int32_t* out = wv == 0 ? P.co_a : P.co_c;
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
        if (wv == 0 && lane == 0 && P.co_pair != nullptr) P.co_pair[g] = static_cast<float>(pc);
      } else {
        // DyGFormer counts on A' = [node_a] ++ A, C' = [node_c] ++ C (length K+1)
        const int32_t na0 = static_cast<int32_t>(query_node(P, qa));
        const int32_t nc0 = static_cast<int32_t>(query_node(P, qc));
        const int L = K + 1;
        int32_t* out = wv == 0 ? P.co_a : P.co_c;
        if (wv == 0 && P.co_pair != nullptr) {
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
        for (int i = lane; i < L; i += kWave) {
          const int32_t ai = i == 0 ? na0 : A[i - 1];
          const int32_t ci = i == 0 ? nc0 : Cc[i - 1];
          int f0 = 0, f1 = 0;
          if (wv == 0) {
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
  }
}

// stand-alone co-occurrence (FREQ) over id rows: one wavefront per pair
__global__ __launch_bounds__(64) void co_occurrence_rows(const int32_t* __restrict__ a_ids,
                                                         const int32_t* __restrict__ c_ids,
                                                         int64_t pairs, int K,
                                                         int32_t* __restrict__ a_cnt,
                                                         int32_t* __restrict__ c_cnt,
                                                         float* __restrict__ pair_count) {
  extern __shared__ int32_t rows[];
  int32_t* A = rows;
  int32_t* Cc = rows + K;
  const int64_t g = blockIdx.x;
  const int lane = threadIdx.x;
  for (int i = lane; i < K; i += kWave) {
    A[i] = a_ids[g * K + i];
    Cc[i] = c_ids[g * K + i];
  }
  __syncthreads();
  int pc = 0;
  for (int i0 = 0; i0 < K; i0 += kWave) {
    const int i = i0 + lane;
    int aa = 0, ac = 0, ca = 0, cc = 0;
    int32_t x = -1, y = -1;
    if (i < K) {
      x = A[i];
      y = Cc[i];
      for (int j = 0; j < K; ++j) {
        const int32_t aj = A[j], cj = Cc[j];
        aa += aj == x;
        ac += cj == x;
        ca += aj == y;
        cc += cj == y;
      }
      if (x == -1) aa = ac = 0;
      if (y == -1) ca = cc = 0;
      a_cnt[(g * K + i) * 2 + 0] = aa;
      a_cnt[(g * K + i) * 2 + 1] = ac;
      c_cnt[(g * K + i) * 2 + 0] = ca;
      c_cnt[(g * K + i) * 2 + 1] = cc;
    }
    pc += __popcll(__ballot(i < K && x != -1 && ac > 0));
  }
  if (lane == 0 && pair_count != nullptr) pair_count[g] = static_cast<float>(pc);
}

int round16(int x) { return (x + 15) & ~15; }

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_recent(const tgx_ring* ring, const tgx_csr* csr, const tgx_recent_args* a,
                          void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (a == nullptr) return fail(TGX_ERR_ARG, "tgx_recent: args is NULL");
  if (a->num_queries < 0 || a->num_groups < 0)
    return fail(TGX_ERR_ARG, "tgx_recent: negative query/group count");
  if (a->k < 1 || a->k > TGX_MAX_K)
    return fail(TGX_ERR_LIMIT, "tgx_recent: k=%d outside [1, %d]", a->k, TGX_MAX_K);
  if (a->group < 1 || a->group > TGX_MAX_GROUP)
    return fail(TGX_ERR_LIMIT, "tgx_recent: group=%d outside [1, %d]", a->group, TGX_MAX_GROUP);
  if (a->num_groups >= (int64_t(1) << 31))
    return fail(TGX_ERR_LIMIT, "tgx_recent: too many groups");
  if (a->num_queries == 0 || a->num_groups == 0) return TGX_OK;
  if (a->num_query_groups < 0 || a->num_query_groups > TGX_MAX_QUERY_GROUPS)
    return fail(TGX_ERR_LIMIT, "tgx_recent: %d query groups outside [0, %d]", a->num_query_groups,
                TGX_MAX_QUERY_GROUPS);
  if ((a->num_query_groups == 0 && (a->nodes == nullptr || a->times == nullptr)) ||
      a->out_ids == nullptr || a->out_times == nullptr || a->out_mask == nullptr)
    return fail(TGX_ERR_ARG, "tgx_recent: nodes/times/out_ids/out_times/out_mask must not be NULL");
  if (a->plan == nullptr && a->num_groups * a->group < a->num_queries)
    return fail(TGX_ERR_ARG, "tgx_recent: num_groups*group < num_queries without a plan");

  Params P{};
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
    P.c_off = csr->offsets;
    P.c_ids = csr->ids;
    P.c_times = csr->times;
    P.c_feats = static_cast<const uint8_t*>(csr->feats);
    P.c_eids = csr->eids;
    feat_dim = csr->feat_dim;
    dtype = csr->feat_dtype;
  }
  if (ring == nullptr && csr == nullptr) {
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
    for (int g = 0; g < a->num_query_groups; ++g) {
      const tgx_query_group& qg = a->query_groups[g];
      if (qg.count < 0 || qg.times_per < 1 || (qg.count > 0 && (qg.nodes == nullptr || qg.times == nullptr)))
        return fail(TGX_ERR_ARG, "tgx_recent: bad query group %d", g);
      P.gn[g] = qg.nodes;
      P.gt[g] = qg.times;
      P.gdiv[g] = qg.times_per;
      P.goff[g] = off;
      off += qg.count;
    }
    P.goff[a->num_query_groups] = off;
    if (a->num_query_groups > 0 && off != a->num_queries)
      return fail(TGX_ERR_ARG, "tgx_recent: query groups hold %lld queries, num_queries is %lld",
                  (long long)off, (long long)a->num_queries);
  }
  P.Q = a->num_queries;
  P.K = a->k;
  P.plan = a->plan;
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
  P.dt_mode = a->dt_mode;
  P.o_te = a->out_te;
  P.te_vec4 = (a->d_t % 4 == 0 && aligned16(a->out_te)) ? 1 : 0;
  if (a->co_mode != TGX_CO_NONE && a->co_mode != TGX_CO_FREQ && a->co_mode != TGX_CO_DYGFORMER)
    return fail(TGX_ERR_ARG, "tgx_recent: unknown co_mode %d", a->co_mode);
  if (a->co_mode != TGX_CO_NONE && (a->group < 2 || a->co_a == nullptr || a->co_c == nullptr))
    return fail(TGX_ERR_ARG, "tgx_recent: co-occurrence needs group >= 2 and co_a/co_c");
  P.co_mode = a->co_mode;
  P.co_a = a->co_a;
  P.co_c = a->co_c;
  P.co_pair = a->co_pair;
  P.status = a->status;

  const int K = a->k;
  P.cand_cap = K + P.B;
  P.te_bytes = 2 * round16(a->d_t * 4);
  P.wave_bytes = round16(P.cand_cap * 16 + K * 12);
  const size_t lds = static_cast<size_t>(P.te_bytes) + static_cast<size_t>(a->group) * P.wave_bytes;
  if (lds > 160 * 1024) return fail(TGX_ERR_LIMIT, "tgx_recent: %zu bytes of LDS needed", lds);

  int vec = 2;
  const bool fe = a->out_feats != nullptr && P.row_bytes > 0;
  auto al = [](const void* p, unsigned m) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & m) == 0; };
  if (P.row_bytes % 16 == 0 && (!fe || (al(P.r_feats, 15) && al(P.c_feats, 15) && al(P.o_feats, 15))))
    vec = 16;
  else if (P.row_bytes % 4 == 0 && (!fe || (al(P.r_feats, 3) && al(P.c_feats, 3) && al(P.o_feats, 3))))
    vec = 4;

  hipEvent_t ev0 = static_cast<hipEvent_t>(a->timing_start);
  hipEvent_t ev1 = static_cast<hipEvent_t>(a->timing_stop);
  if ((ev0 == nullptr) != (ev1 == nullptr))
    return fail(TGX_ERR_ARG, "tgx_recent: timing_start and timing_stop must both be set or both NULL");
  const dim3 grid(static_cast<unsigned>(a->num_groups));
  const dim3 block(kWave * a->group);
  static bool attr_done = false;
  if (!attr_done) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(recent_fused<16>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(recent_fused<4>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(recent_fused<2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipGetLastError();
    attr_done = true;
  }
  switch (vec) {
    case 16:
      hipExtLaunchKernelGGL(recent_fused<16>, grid, block, lds, stream, ev0, ev1, 0, P);
      break;
    case 4:
      hipExtLaunchKernelGGL(recent_fused<4>, grid, block, lds, stream, ev0, ev1, 0, P);
      break;
    default:
      hipExtLaunchKernelGGL(recent_fused<2>, grid, block, lds, stream, ev0, ev1, 0, P);
      break;
  }
  return check_launch("recent_fused");
}

extern "C" int tgx_co_occurrence(const int32_t* a_ids, const int32_t* c_ids, int64_t pairs,
                                 int32_t k, int32_t* a_cnt, int32_t* c_cnt, float* pair_count,
                                 void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (pairs < 0 || k < 0) return fail(TGX_ERR_ARG, "tgx_co_occurrence: negative size");
  if (k > 4096) return fail(TGX_ERR_LIMIT, "tgx_co_occurrence: k=%d above 4096", k);
  if (pairs >= (int64_t(1) << 31)) return fail(TGX_ERR_LIMIT, "tgx_co_occurrence: too many pairs");
  if (pairs == 0 || k == 0) return TGX_OK;
  if (a_ids == nullptr || c_ids == nullptr || a_cnt == nullptr || c_cnt == nullptr)
    return fail(TGX_ERR_ARG, "tgx_co_occurrence: NULL pointer");
  hipLaunchKernelGGL(co_occurrence_rows, dim3(static_cast<unsigned>(pairs)), dim3(kWave),
                     2 * k * sizeof(int32_t), stream, a_ids, c_ids, pairs, k, a_cnt, c_cnt,
                     pair_count);
  return check_launch("co_occurrence_rows");
}
