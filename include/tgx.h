/*
 * tgx.h -- C ABI of libtgx.so, the MI355X (gfx950) fused temporal data pipeline.
 *
 * Plain C: device pointers, sizes, dtype enums and a HIP stream passed as
 * `void*` (a hipStream_t; NULL means the legacy default stream).  No torch
 * types cross this boundary.  Every entry point:
 *   - launches only on the given stream and never synchronises the device;
 *   - never allocates or frees device memory: outputs, ring arrays and the
 *     workspace belong to the caller;
 *   - keeps no state between calls (safe from any host thread);
 *   - returns TGX_OK (0) or an error code; the message of the last failure on
 *     the calling thread is returned by tgx_last_error().
 *
 * Reference interfaces replaced (paths relative to the tgengine checkout):
 *   tgx_ring_append   <- TemporalGraph.advance post-freeze branch
 *                        tgengine/core/temporal_graph.py:123-129 and
 *                        _append_overflow :351-387 (pure torch there; no native op);
 *                        tgx_ring_plan / tgx_ring_commit / tgx_ring_discard split it
 *   tgx_recent        <- TemporalGraph.recent :183-349 (ring merge _merge_overflow
 *                        :307-349, CSR window :241-305) and the pybind op
 *                        temporal_recent_k (tgengine/core/csrc/temporal_sample.cu:291-329,
 *                        bound at :546-555 via tgengine/core/kernels.py:135-154), fused
 *                        with FixedCosineTimeEncoder (tgengine/nn/time_encoding.py:37-63)
 *                        and DyGFormer co-occurrence counting
 *                        (tgengine/models/dygformer.py:71-87)
 *   tgx_co_occurrence <- pybind op co_occurrence_freq (temporal_sample.cu:514-543,
 *                        kernels.py:203-221) and the (B,) pair count of
 *                        DataPipeline._co_occur_from_neighbors
 *                        (tgengine/pipeline/__init__.py:206-219)
 */
#ifndef TGX_H
#define TGX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGX_ABI_VERSION 17

/* status codes */
#define TGX_OK 0
#define TGX_ERR_ARG 1      /* bad argument (null pointer, negative size, ...) */
#define TGX_ERR_DTYPE 2    /* unsupported dtype */
#define TGX_ERR_LIMIT 3    /* size beyond a documented limit */
#define TGX_ERR_HIP 4      /* a HIP runtime call failed (message has the HIP error) */

/* feature storage dtypes */
#define TGX_F32 0
#define TGX_BF16 1

/* dt conventions of the time encoding */
#define TGX_DT_DYGFORMER 0 /* dt = f32(q) - f32(t) in fp32; padding slots encode to 0 */
#define TGX_DT_TGN 1       /* dt = f32(q - t) (float64 subtract); padding uses t = 0.0 */

/* co-occurrence modes (pairs = queries 0 and 1 of every plan group) */
#define TGX_CO_NONE 0
#define TGX_CO_FREQ 1      /* int32 (P,K,2) counts per sequence + (P,) pair count */
#define TGX_CO_DYGFORMER 2 /* int32 (P,1+K,2): DyGFormer counts with the node at pos 0 */

/* device-side diagnostics: int32 status[TGX_STATUS_WORDS], accumulated */
#define TGX_STATUS_WORDS 8
#define TGX_ST_BAD_EVENT_NODE 0   /* append: src/dst outside [0, num_nodes) (entry skipped) */
#define TGX_ST_KEY_COLLISION 1    /* append: int(max t)+2 <= 2b-1 (reference key not lexicographic) */
#define TGX_ST_BAD_QUERY_NODE 2   /* recent: query node >= num_nodes (query returns padding) */

/* Per-node ring of `slots` entries (reference: temporal_graph.py:89-102).
 * ids int32 [N,B] (-1 empty), times float64 [N,B], feats [N,B,feat_dim] of
 * feat_dtype, write_pos int64 [N], eids int64 [N,B] (optional, may be NULL).
 * scratch: tgx_ring_scratch_size(N) bytes of device memory, zero-filled once by
 * the caller before the first append and otherwise left to the library: its
 * first N int32 are per-node counters that every tgx_ring_append restores to
 * zero, the rest is rewritten before each use.  Needed by tgx_ring_append only
 * (tgx_recent ignores it). */
typedef struct tgx_ring {
  int64_t num_nodes;
  int32_t slots;
  int32_t feat_dim;
  int32_t feat_dtype;
  int32_t reserved;
  int32_t* ids;
  double* times;
  void* feats;
  int64_t* write_pos;
  int64_t* eids;
  int32_t* scratch;
} tgx_ring;

/* Frozen CSR (reference: temporal_graph.py:133-181): offsets int64 [N+1],
 * ids int32 [E], times float64 [E] (ascending within a node), feats [E,feat_dim],
 * eids int64 [E] (optional).  max_time: the largest non-NaN time of the entries
 * (+inf when unknown).  Results never depend on it: a query at a later time is
 * after every window, and the gather then skips the search work it would issue
 * ahead for a query that may fall inside one. */
typedef struct tgx_csr {
  int64_t num_nodes;
  int64_t num_entries;
  int32_t feat_dim;
  int32_t feat_dtype;
  const int64_t* offsets;
  const int32_t* ids;
  const double* times;
  const void* feats;
  const int64_t* eids;
  double max_time;
} tgx_csr;

/* One group of queries read in place: query l of the group is node nodes[l]
 * at time times[l / times_per] (times_per = negatives per event for a (b, n)
 * row-major negative block, else 1). */
typedef struct tgx_query_group {
  const void* nodes;       /* [count] node ids: int64, or int32 with TGX_QG_NODES_I32 */
  const double* times;
  int64_t count;
  int32_t times_per;
  int32_t flags;           /* TGX_QG_* bits */
  const uint8_t* valid;    /* [count] or NULL; a 0 makes that query padding only
                              (no candidates, no status count): the 2-hop queries
                              under invalid hop-1 slots */
} tgx_query_group;
#define TGX_QG_NODES_I32 1

/* work plans of tgx_recent_args.plan_mode */
#define TGX_PLAN_TILES 0
#define TGX_PLAN_EVENTS 1
#define TGX_PLAN_LIST 2

#define TGX_MAX_QUERY_GROUPS 4

typedef struct tgx_recent_args {
  /* queries: either nodes/times, or num_query_groups > 0 groups concatenated
   * in order (query index = group offset + position in the group) */
  const int64_t* nodes;    /* [Q] node ids; < 0 = padding query */
  const double* times;     /* [Q] query times */
  int64_t num_queries;
  int32_t k;               /* neighbours per query, 1..TGX_MAX_K */
  /* work plan, by plan_mode:
   *   TGX_PLAN_TILES (plan NULL): consecutive queries; `group` queries per
   *     workgroup (a hint: when a small launch shares each query among several
   *     wavefronts, a query takes a workgroup of its own); num_groups is ignored;
   *   TGX_PLAN_EVENTS (plan NULL): event-major groups computed from the query
   *     groups: group g = event g holds, for each query group in order,
   *     its times_per queries of event g (the reference grouping [src, dst,
   *     neg row-major, neg_src], pipeline/__init__.py:40-70, read as one
   *     group per event); group = sum of times_per, num_groups = events.
   *     With event_query_groups = E > 0, only the first E query groups form
   *     the events (group = their sum of times_per); the queries of the other
   *     groups follow in workgroups of `group` consecutive queries;
   *   TGX_PLAN_LIST (plan set): group g handles queries plan[g*group + j],
   *     j < group (-1 = none).
   * Co-occurrence needs TGX_PLAN_EVENTS or TGX_PLAN_LIST (its pairs are
   * queries 0 and 1 of a group). */
  const int32_t* plan;
  int32_t group;           /* 1..8 */
  int32_t plan_mode;       /* TGX_PLAN_*; TGX_PLAN_LIST iff plan != NULL */
  int64_t num_groups;
  /* outputs (row = query index); out_feats / out_eids / out_te may be NULL */
  int32_t* out_ids;        /* [Q,K] */
  double* out_times;       /* [Q,K] */
  void* out_feats;         /* [Q,K,feat_dim] in the storage dtype */
  uint8_t* out_mask;       /* [Q,K] 0/1 */
  int64_t* out_eids;       /* [Q,K] */
  /* fused FixedCosineTimeEncoder: out_te[Q,K,d_t] = cos(fl32(dt*w) [+ b]) */
  int32_t d_t;             /* 0 = off */
  const float* te_w;       /* [d_t] */
  const float* te_b;       /* [d_t] or NULL (bias 0) */
  int32_t dt_mode;         /* TGX_DT_* */
  float* out_te;
  /* fused co-occurrence for the (query 0, query 1) pair of every group */
  int32_t co_mode;         /* TGX_CO_* */
  int32_t* co_a;           /* FREQ: [P,K,2]; DYGFORMER: [P,1+K,2] */
  int32_t* co_c;
  float* co_pair;          /* [P] float shared-neighbour count (both modes), may be NULL */
  int32_t* status;         /* [TGX_STATUS_WORDS] or NULL */
  int32_t num_query_groups;                          /* 0 = use nodes/times */
  tgx_query_group query_groups[TGX_MAX_QUERY_GROUPS];
  /* optional hipEvent_t pair recorded by the kernel dispatch itself (start and
   * end of the kernel's execution); both NULL = plain launch */
  void* timing_start;
  void* timing_stop;
  /* optional ring plan run by the same launch (append_b > 0): tgx_ring_plan of
   * the batch append_src/dst/time (append_b events, append_workspace of
   * tgx_ring_append_workspace_size(append_b) bytes) that the caller appends
   * next, through tgx_ring_commit (or drops through tgx_ring_discard).  The plan
   * reads the batch and the ring's write positions and writes only the
   * workspace, so it runs beside the gather; batches above 16384 events are
   * planned by launches of their own after the gather.  append_b == 0: no plan. */
  const int64_t* append_src;
  const int64_t* append_dst;
  const double* append_time;
  int64_t append_b;
  void* append_workspace;
  size_t append_workspace_bytes;
  /* TGX_PLAN_EVENTS: the number of leading query groups that form the events
   * (0 = all of them; see plan_mode) */
  int32_t event_query_groups;
  /* d_t > 0: upper bounds of max|te_w[i]| and max|te_b[i]| (0 without bias),
   * which let the cosine skip its large-argument reduction where no argument
   * can need it.  te_bound_w <= 0 (or NaN): unknown, every element takes the
   * full-range reduction (same results, slower).  The bounds are trusted and
   * not checked on the device: a bound below the true maximum gives WRONG
   * encodings (errors far above 1e-6) wherever |fl32(dt * w) + b| reaches 2^29.
   * Pass 0 unless the bound is known on the host. */
  float te_bound_w;
  float te_bound_b;
} tgx_recent_args;

#define TGX_MAX_SLOTS 64
#define TGX_MAX_K 512
#define TGX_MAX_GROUP 8
#define TGX_MAX_DT 512

/* Ring update for one batch of b undirected events (kernel a).
 * Entries are the 2b directed edges in the order [src->dst ..., dst->src ...];
 * per node the last min(c, B) entries in that order are written to slots
 * (write_pos + m) % B, m = 0.., and write_pos grows by min(c, B).
 * feat: [b, feat_dim] in ring->feat_dtype, or NULL for zero features.
 * eids (if the ring has them) receive eid_base + event index.
 * workspace: tgx_ring_append_workspace_size(b) bytes of device memory, 16-byte
 * aligned (no initialisation needed).  Calls on one ring must be ordered (one
 * stream). */
int tgx_ring_append(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                    const double* time, const void* feat, int64_t b, int64_t eid_base,
                    void* workspace, size_t workspace_bytes, int32_t* status, void* stream);
size_t tgx_ring_append_workspace_size(int64_t b);
size_t tgx_ring_scratch_size(int64_t num_nodes);

/* tgx_ring_append with no workspace argument and no allocation: the workspace is
 * a file-scope device array of tgx_ring_append_static_max_bytes() bytes (2 MiB;
 * each GPU the library runs on holds its own copy until the process ends),
 * enough for batches with tgx_ring_append_workspace_size(b) <= that (about
 * 100,000 events); larger batches return TGX_ERR_LIMIT.  It calls no hipMalloc
 * or hipFree.  Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race; calls ordered on one
 * stream are safe.  The ring's scratch is the caller's, as for tgx_ring_append.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). */
int tgx_ring_append_static(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                           const double* time, const void* feat, int64_t b, int64_t eid_base,
                           int32_t* status, void* stream);
size_t tgx_ring_append_static_max_bytes(void);

/* tgx_ring_append in two halves, so the first can run while other work still
 * reads the ring (the same split of _append_overflow, temporal_graph.py:351-387):
 *   tgx_ring_plan   : up to 16384 events, every entry's slot (or none) and every
 *                     node's new write position, in the workspace; reads
 *                     src/dst/time and write_pos, writes no ring array and no
 *                     scratch but two diagnostic words.  Above 16384 events,
 *                     per-node counts and entry lists in the workspace and the
 *                     ring's scratch, reading src/dst/time only; needs the
 *                     scratch counters at zero (as every commit or discard
 *                     leaves them).
 *   tgx_ring_commit : the ring writes of a planned batch (same arguments and
 *                     workspace as its plan); restores the counters; reports the
 *                     plan's diagnostics into `status`.
 *   tgx_ring_discard: drops a planned batch without touching the ring arrays and
 *                     restores the counters.
 * Plan, then exactly one of commit / discard, ordered on streams by the caller,
 * with no other write to the ring between them (the plan reads write_pos). */
int tgx_ring_plan(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                  const double* time, int64_t b, void* workspace, size_t workspace_bytes,
                  void* stream);
int tgx_ring_commit(const tgx_ring* ring, const int64_t* src, const int64_t* dst,
                    const double* time, const void* feat, int64_t b, int64_t eid_base,
                    void* workspace, size_t workspace_bytes, int32_t* status, void* stream);
int tgx_ring_discard(const tgx_ring* ring, const int64_t* src, const int64_t* dst, int64_t b,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Frozen-CSR build (TemporalGraph.freeze_csr, temporal_graph.py:133-181).
 * The n directed entries of the pre-freeze advance() calls, in build order
 * (per call: [src->dst for every event, dst->src for every event]), are sorted
 * stably by time, then stably by node: a node's entries end up time-ascending
 * with ties in build order.  Outputs (the tgx_csr arrays): out_offsets [N+1],
 * out_ids int32 [n] (= to), out_times [n], out_feats [n, feat_dim] (row of the
 * entry's event in feats, zero when feats is NULL), out_eids [n] (= event, may
 * be NULL).  Entries whose node is outside [0, N), or whose event is outside
 * [0, num_events) while feats is set, are counted in
 * status[TGX_ST_BAD_EVENT_NODE] (out-of-range nodes sort after every node).
 * workspace: tgx_csr_build_workspace_size(n) bytes, no initialisation needed.
 *
 * flags & TGX_CSR_EVENT_PAIRS: from/to/time hold the n/2 EVENTS (src, dst,
 * time) instead of the n entries, in an order where the stable sort by time
 * is the identity on the entries 2k = from[k]->to[k], 2k+1 = to[k]->from[k]
 * (both at time[k]; event index k, or event[k] when event is set): times
 * strictly increasing within every advance() call and non-decreasing across
 * calls, which makes this order the stable time order of the build order.  The
 * time passes are skipped; the caller checks the condition.
 *
 * flags & TGX_CSR_EVENTS_BY_CALL: from/to/time (and event) hold the n/2
 * events in stream order, and call_starts [num_calls] the first event of each
 * advance() call (ascending, starting at 0); the build forms the build order
 * itself (per call: from->to of each event, then to->from of each) and sorts
 * it by time.  With TGX_CSR_NONDECREASING as well, the caller asserts that
 * time never decreases along the events (no NaN): the stable time order is
 * then, run by run of equal times within a call, the run's from->to entries
 * followed by its to->from entries, and the time passes are skipped.  Call
 * starts outside [1, n/2) are ignored; a wrong order assertion gives a wrong
 * order, never an access outside the arrays. */
typedef struct tgx_csr_build_args {
  int64_t num_nodes;
  int64_t num_entries;
  const int64_t* from;     /* [n] node of each entry */
  const int64_t* to;       /* [n] neighbour id */
  const double* time;      /* [n] */
  const int64_t* event;    /* [n] event of each entry: edge id and feature row (NULL when unused) */
  const void* feats;       /* [num_events, feat_dim] in feat_dtype, or NULL */
  int64_t num_events;
  int32_t feat_dim;
  int32_t feat_dtype;
  int64_t* out_offsets;
  int32_t* out_ids;
  double* out_times;
  void* out_feats;
  int64_t* out_eids;
  void* workspace;
  size_t workspace_bytes;
  int32_t* status;         /* [TGX_STATUS_WORDS] or NULL */
  uint32_t flags;          /* TGX_CSR_* */
  const int64_t* call_starts;  /* [num_calls], TGX_CSR_EVENTS_BY_CALL only */
  int64_t num_calls;
} tgx_csr_build_args;

#define TGX_CSR_EVENT_PAIRS 1u
#define TGX_CSR_EVENTS_BY_CALL 2u
#define TGX_CSR_NONDECREASING 4u

size_t tgx_csr_build_workspace_size(int64_t num_entries);
int tgx_csr_build(const tgx_csr_build_args* args, void* stream);

/* Pre-freeze scan.  No counterpart in the reference, whose freeze_csr
 * (temporal_graph.py:133-181) sorts host lists; here freeze_csr learns from it,
 * in one round trip, the node range it checks, which build to run (event pairs
 * or general) and the largest time.  Over the num_events > 0 events src/dst/time of the pre-freeze
 * advance() calls, whose first events are call_starts [num_calls] (ascending,
 * a repeated value counts once; may be NULL when num_calls is 0), writes out
 * int64 [4]:
 *   out[0], out[1]  min and max node id over src and dst,
 *   out[2]          2 when the stream is time-ordered in the sense of
 *                   TGX_CSR_EVENT_PAIRS: for every k >= 1 the float64
 *                   difference time[k] - time[k-1] is > 0, or == 0 with k in
 *                   call_starts (NaN and inf - inf differences break it);
 *                   else 1 when time[k] >= time[k-1] for every k >= 1 (the
 *                   TGX_CSR_NONDECREASING condition), else 0,
 *   out[3]          the bits of the largest non-NaN time (-inf when all are NaN).
 * workspace: tgx_csr_scan_workspace_size() bytes, no initialisation needed.
 * Two launches; the caller reads out after the stream. */
size_t tgx_csr_scan_workspace_size(void);
int tgx_csr_scan(const int64_t* src, const int64_t* dst, const double* time, int64_t num_events,
                 const int64_t* call_starts, int64_t num_calls, int64_t* out, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Historical negative pool (HistoricalNegPool, pipeline/negatives.py:14-126).
 * pool int32 [num_nodes, pool_size] (-1 = empty), count int64 [num_nodes]
 * (edges seen per source), both zero-/minus-one-filled by the caller once.
 * update: edge j of the batch, the r-th from its source u in batch order, is
 * u's e-th edge (e = count[u] + r + 1): e <= pool_size fills slot e-1, else it
 * replaces slot rand % pool_size with probability pool_size/e (float32); the
 * later edge of the batch wins a slot two edges take; count[u] grows by u's
 * edges.  sample: out[q] = pool[u][int(U * min(count[u], pool_size))] (slot
 * clamped to pool_size-1), or a random node in [0, num_nodes) for a node with
 * no history.  Random numbers: rand64(seed, call, i, stream) =
 * mix(mix(mix(seed ^ 0x9e3779b97f4a7c15) ^ call) ^ (4i + stream)), mix the
 * splitmix64 finalizer, U = (rand64 >> 40) * 2^-24; streams 0/1 (update accept /
 * slot), 2/3 (sample slot / fallback node).  Out-of-range ids are skipped
 * (update) or sampled as nodes without history (sample) and counted in status.
 * workspace: tgx_negpool_update_workspace_size(n) bytes (no initialisation
 * needed).  scratch: NULL, or tgx_negpool_scratch_size() bytes of device memory,
 * 256-byte aligned, zero-filled once by the caller and otherwise left to the
 * library (a table that every update leaves zeroed again); with it, batches of
 * up to 32,768 edges update in two launches over the whole device, without it in
 * one workgroup (up to 8,192 edges) or by sorting.  Same results either way.
 * Updates that share a scratch must be ordered (one stream). */
size_t tgx_negpool_update_workspace_size(int64_t n);
size_t tgx_negpool_scratch_size(void);
int tgx_negpool_update(int32_t* pool, int64_t* count, int64_t num_nodes, int32_t pool_size,
                       const int64_t* src, const int64_t* dst, int64_t n, uint64_t seed,
                       uint64_t call, void* workspace, size_t workspace_bytes, void* scratch,
                       size_t scratch_bytes, int32_t* status, void* stream);
int tgx_negpool_sample(const int32_t* pool, const int64_t* count, int64_t num_nodes,
                       int32_t pool_size, const int64_t* src, int64_t n, uint64_t seed,
                       uint64_t call, int64_t* out, int32_t* status, void* stream);

/* The same two operations with the caller's random draws, indexed as the
 * reference indexes its torch.rand / torch.randint draws
 * (pipeline/negatives.py:78-86, :116-124), so that draws taken from torch's
 * generator in the reference's call order give the reference's pool and
 * samples.  update: u_accept[p] (float32 in [0, 1)) and slot_draw[p] (in
 * [0, pool_size); other values skip the edge) of the edge at position p of
 * the batch's stable sort by source; sample: u_slot[q] (float32 in [0, 1)) of
 * query q, and out[q] = -1 for a node without history (the reference then
 * draws those nodes with torch.randint(0, num_nodes, (#such queries,)) in
 * query order; the caller does that).  The later edge of a batch still wins a
 * slot two accepted edges take, where the reference leaves it to the last
 * index_put_ write. */
int tgx_negpool_update_draws(int32_t* pool, int64_t* count, int64_t num_nodes, int32_t pool_size,
                             const int64_t* src, const int64_t* dst, int64_t n,
                             const float* u_accept, const int64_t* slot_draw, void* workspace,
                             size_t workspace_bytes, int32_t* status, void* stream);
int tgx_negpool_sample_draws(const int32_t* pool, const int64_t* count, int64_t num_nodes,
                             int32_t pool_size, const int64_t* src, int64_t n, const float* u_slot,
                             int64_t* out, int32_t* status, void* stream);

/* Fused most-recent-K gather (+ time encoding, + co-occurrence) (kernels b, c).
 * ring and/or csr may be NULL (no candidates from that store); with both NULL
 * every query is padding and out_feats must be NULL (the row width comes from
 * them). */
int tgx_recent(const tgx_ring* ring, const tgx_csr* csr, const tgx_recent_args* args,
               void* stream);

/* Launch shape tgx_recent would use for these arguments, without launching:
 * shape[0] workgroups, [1] threads per workgroup, [2] dynamic LDS bytes,
 * [3] queries per wavefront, [4] wavefronts per query in one workgroup (a
 * query split over more than 4 wavefronts without a ring spreads them over
 * several workgroups), [5] queries per workgroup (1 also for those),
 * [6] plan workgroups, [7] feature copy width in bytes.  Same
 * argument checks and return codes as tgx_recent. */
int tgx_recent_launch_shape(const tgx_ring* ring, const tgx_csr* csr, const tgx_recent_args* args,
                            int64_t shape[8]);

/* Stand-alone co-occurrence over neighbour-id rows a, c int32 [P,K]:
 * a_cnt/c_cnt int32 [P,K,2] (mode FREQ) and pair_count float [P] (may be NULL).
 * a_mask / c_mask uint8 [P,K] (0/1) mark the valid positions; with a NULL mask
 * a position is valid iff its id is not -1.  A count covers valid positions
 * only, and an invalid position's counts are 0 (reference
 * temporal_sample.cu:453-511, and the masked pair count of
 * pipeline/__init__.py:206-219). */
int tgx_co_occurrence(const int32_t* a_ids, const int32_t* c_ids, const uint8_t* a_mask,
                      const uint8_t* c_mask, int64_t pairs, int32_t k, int32_t* a_cnt,
                      int32_t* c_cnt, float* pair_count, void* stream);

const char* tgx_last_error(void);
int tgx_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TGX_H */
