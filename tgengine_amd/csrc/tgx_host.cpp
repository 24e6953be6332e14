// Host glue of the Python API (torch extension module `tgengine_amd._tgx_host`).
//
// One call per TemporalGraph.recent / DataPipeline.prepare / advance: it checks
// the inputs, allocates the outputs from the caching allocator, fills the C-ABI
// argument block, launches through libtgx and returns the per-group tensors.
// All device work is in libtgx (include/tgx.h), which never sees a torch type.
//
// The outputs of one launch live in two allocations (two caching-allocator
// round trips per prepare): a small block with ids, times, masks, edge ids and
// co-occurrence counts, and a bulk block with the feature rows and time
// encodings.  The per-group tensors are typed blocks of those byte buffers,
// built directly as TensorImpls: they share the buffer's storage and are plain
// tensors, not autograd views of each other.  Keeping one tensor alive keeps
// its whole block alive, so a caller that keeps only masks or ids does not pin
// the feature rows and encodings.
//
// The per-batch calls of the streaming loop (Prepare.run, PlanSlot.commit) read
// the caller's current HIP stream themselves and hand their tensors straight to
// Python, so one step costs two calls into this module.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "tgx.h"

namespace py = pybind11;

namespace {

// Event-major launches (co-occurrence) of at most this many queries group only the
// (src, dst) pair of each event and tile the other query groups after them, so that
// more wavefronts share each query (a workgroup holds at most 8 wavefronts: query
// slots x split); larger launches keep every query of an event in its group unless
// an event holds more queries than a workgroup takes (TGX_MAX_GROUP, or the
// waves whose LDS fits the CU at this k), when they too group only the pair
constexpr int64_t kPairTailMaxQueries = 4096;

// an upper bound of one wave's LDS in tgx_recent at k neighbours (k CSR
// candidates and up to 64 ring slots, k ranked positions) plus the encoder weights
int64_t group_lds_bound(int64_t G, int64_t k) { return G * ((k + 64) * 16 + k * 28 + 64) + 4096; }

// event_query_groups of an event-major launch over ng query groups, Q queries,
// G queries per event and k neighbours
int pair_tail_groups(size_t ng, int64_t Q, int64_t G, int64_t k) {
  const bool big = G > TGX_MAX_GROUP || group_lds_bound(G, k) > 160 * 1024;
  return ng > 2 && (Q <= kPairTailMaxQueries || big) ? 2 : 0;
}

void check(int rc, const char* what) {
  if (rc != TGX_OK) throw std::runtime_error(std::string(what) + " failed: " + tgx_last_error());
}

at::Tensor as_dev(const at::Tensor& t, at::ScalarType dt, const at::Device& dev) {
  if (t.scalar_type() == dt && t.device() == dev && t.is_contiguous()) return t;
  return t.to(dev, dt).contiguous();
}

// 1-D view of t (t itself when it already is 1-D)
at::Tensor flat(const at::Tensor& t) { return t.dim() == 1 ? t : t.reshape({-1}); }

// a contiguous `st` tensor of shape `sizes` at byte offset `byte_off` of base's
// storage (a multiple of the element size)
at::Tensor typed_block(const at::Tensor& base, const caffe2::TypeMeta dt, int64_t byte_off,
                       at::IntArrayRef sizes) {
  auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(base.storage()), base.key_set(), dt);
  impl->set_sizes_contiguous(sizes);
  impl->set_storage_offset(byte_off / static_cast<int64_t>(dt.itemsize()));
  return at::Tensor(std::move(impl));
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// the caller's current stream on device `index`, as tgx takes it
void* current_stream(c10::DeviceIndex index) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(index).stream());
}

// identity of a tensor for the plan check: the same tensor, or a view of the
// same memory with the same shape, strides and dtype
bool same_tensor(const at::Tensor& a, const at::Tensor& b) {
  if (a.unsafeGetTensorImpl() == b.unsafeGetTensorImpl()) return true;
  return a.data_ptr() == b.data_ptr() && a.sizes() == b.sizes() && a.strides() == b.strides() &&
         a.scalar_type() == b.scalar_type();
}

uint32_t version_of(const at::Tensor& t) {
  return t.unsafeGetTensorImpl()->version_counter().current_version();
}

// Byte layout of the outputs of one tgx_recent launch over Q queries: the bulk
// block (feature rows, encodings) and the small block (times, edge ids, ids,
// co-occurrence, masks), every field 256-byte aligned within its block.
struct Layout {
  int64_t feats = 0, te = 0, bulk = 0;
  int64_t times = 0, eids = 0, ids = 0, coa = 0, coc = 0, cop = 0, mask = 0, small = 0;
  Layout(int64_t Q, int64_t k, int64_t row_bytes, int64_t d_t, bool want_eids, int64_t co_rows,
         int64_t co_len) {
    const int64_t QK = Q * k;
    int64_t o = 0;
    feats = o;
    o = align256(o + QK * row_bytes);
    te = o;
    o = align256(o + QK * d_t * 4);
    bulk = o;
    o = 0;
    times = o;
    o = align256(o + QK * 8);
    eids = o;
    o = align256(o + (want_eids ? QK * 8 : 0));
    ids = o;
    o = align256(o + QK * 4);
    coa = o;
    o = align256(o + co_rows * co_len * 2 * 4);
    coc = o;
    o = align256(o + co_rows * co_len * 2 * 4);
    cop = o;
    o = align256(o + co_rows * 4);
    mask = o;
    o = align256(o + QK);
    small = o;
  }
};

const caffe2::TypeMeta kI32 = caffe2::TypeMeta::Make<int32_t>();
const caffe2::TypeMeta kI64 = caffe2::TypeMeta::Make<int64_t>();
const caffe2::TypeMeta kF64 = caffe2::TypeMeta::Make<double>();
const caffe2::TypeMeta kF32 = caffe2::TypeMeta::Make<float>();
const caffe2::TypeMeta kBool = caffe2::TypeMeta::Make<bool>();

// the ring plan of a batch can run in the gather launch: int64 / int64 /
// float64 contiguous 1-D tensors of one non-zero length on the launch's device
bool plannable(const at::Tensor& s, const at::Tensor& d, const at::Tensor& t, const at::Device& dev) {
  const int64_t b = s.numel();
  auto ok = [&](const at::Tensor& x, at::ScalarType st) {
    return x.defined() && x.dim() == 1 && x.numel() == b && x.scalar_type() == st &&
           x.device() == dev && x.is_contiguous();
  };
  return b > 0 && ok(s, at::kLong) && ok(d, at::kLong) && ok(t, at::kDouble);
}

// Output tensors of one launch: allocation, layout and the argument block's
// output pointers; per-group tensors are built on demand.
struct Out {
  at::Tensor bulk, small;
  Layout lay;
  int64_t k, row_bytes, d_t, feat_dim;
  caffe2::TypeMeta fdt;
  bool eids, co;
  int64_t co_rows, co_len;
  Out(const at::Device& dev, int64_t Q, int64_t k_, int64_t feat_dim_, at::ScalarType feat_dtype,
      int64_t d_t_, bool want_eids, int64_t co_mode, int64_t co_rows_)
      : lay(Q, k_, feat_dim_ * c10::elementSize(feat_dtype), d_t_, want_eids,
            co_mode != TGX_CO_NONE ? co_rows_ : 0, co_mode == TGX_CO_FREQ ? k_ : k_ + 1),
        k(k_), row_bytes(feat_dim_ * c10::elementSize(feat_dtype)), d_t(d_t_), feat_dim(feat_dim_),
        fdt(c10::scalarTypeToTypeMeta(feat_dtype)), eids(want_eids), co(co_mode != TGX_CO_NONE),
        co_rows(co_mode != TGX_CO_NONE ? co_rows_ : 0),
        co_len(co_mode == TGX_CO_FREQ ? k_ : k_ + 1) {
    const auto opt = at::TensorOptions().device(dev).dtype(at::kByte);
    bulk = at::empty({lay.bulk}, opt);
    small = at::empty({lay.small}, opt);
  }
  uint8_t* pb(int64_t off) const { return static_cast<uint8_t*>(bulk.data_ptr()) + off; }
  uint8_t* ps(int64_t off) const { return static_cast<uint8_t*>(small.data_ptr()) + off; }
  void fill(tgx_recent_args& a) const {
    a.out_ids = reinterpret_cast<int32_t*>(ps(lay.ids));
    a.out_times = reinterpret_cast<double*>(ps(lay.times));
    a.out_feats = pb(lay.feats);
    a.out_mask = ps(lay.mask);
    a.out_eids = eids ? reinterpret_cast<int64_t*>(ps(lay.eids)) : nullptr;
    a.out_te = d_t > 0 ? reinterpret_cast<float*>(pb(lay.te)) : nullptr;
    if (co) {
      a.co_a = reinterpret_cast<int32_t*>(ps(lay.coa));
      a.co_c = reinterpret_cast<int32_t*>(ps(lay.coc));
      a.co_pair = reinterpret_cast<float*>(ps(lay.cop));
    }
  }
  // rows [r0, r0 + n) of every per-query output, appended to v:
  // ids, times, feats, mask, [te], [eids]
  void group(std::vector<at::Tensor>& v, int64_t r0, int64_t n) const {
    const int64_t rk = r0 * k;
    v.push_back(typed_block(small, kI32, lay.ids + rk * 4, {n, k}));
    v.push_back(typed_block(small, kF64, lay.times + rk * 8, {n, k}));
    v.push_back(typed_block(bulk, fdt, lay.feats + rk * row_bytes, {n, k, feat_dim}));
    v.push_back(typed_block(small, kBool, lay.mask + rk, {n, k}));
    if (d_t > 0) v.push_back(typed_block(bulk, kF32, lay.te + rk * d_t * 4, {n, k, d_t}));
    if (eids) v.push_back(typed_block(small, kI64, lay.eids + rk * 8, {n, k}));
  }
  void co_out(std::vector<at::Tensor>& v) const {
    v.push_back(typed_block(small, kI32, lay.coa, {co_rows, co_len, 2}));
    v.push_back(typed_block(small, kI32, lay.coc, {co_rows, co_len, 2}));
    v.push_back(typed_block(small, kF32, lay.cop, {co_rows}));
  }
};

// the tensors as one Python tuple
py::tuple as_tuple(std::vector<at::Tensor>& v) {
  py::tuple t(v.size());
  for (size_t i = 0; i < v.size(); ++i)
    t[i] = py::reinterpret_steal<py::object>(THPVariable_Wrap(std::move(v[i])));
  return t;
}

// The ring update planned ahead of its advance() (TemporalGraph.plan_append, or
// the plan run by a gather launch): the batch's src/dst/time tensors, their
// version counters when planned, and the stream the plan was enqueued on.  One
// per ring; it also holds the plan workspace (grown by the Python layer).  Every
// method runs under the GIL, so each is atomic for Python threads.
class PlanSlot {
 public:
  PlanSlot(int64_t ring_addr, const at::Tensor& status, int64_t feat_dim, at::ScalarType feat_dtype)
      : ring_(ring_addr), status_(status), feat_dim_(feat_dim), feat_dtype_(feat_dtype),
        dev_(status.device()) {}

  void set_workspace(const at::Tensor& ws) { ws_ = ws; }
  c10::optional<at::Tensor> workspace() const {
    return ws_.defined() ? c10::optional<at::Tensor>(ws_) : c10::nullopt;
  }
  bool pending() const { return has_; }
  int64_t stream() const { return has_ ? stream_ : 0; }
  void set_stream(int64_t stream) {
    if (has_) stream_ = stream;
  }
  void record(const at::Tensor& s, const at::Tensor& d, const at::Tensor& t, int64_t stream) {
    src_ = s;
    dst_ = d;
    time_ = t;
    ver_[0] = version_of(s);
    ver_[1] = version_of(d);
    ver_[2] = version_of(t);
    stream_ = stream;
    has_ = true;
  }
  bool matches(const at::Tensor& s, const at::Tensor& d, const at::Tensor& t) const {
    return has_ && same_tensor(s, src_) && same_tensor(d, dst_) && same_tensor(t, time_) &&
           version_of(s) == ver_[0] && version_of(d) == ver_[1] && version_of(t) == ver_[2];
  }
  // (src, dst, time, stream) of the pending plan, which is no longer pending; None
  py::object take() {
    if (!has_) return py::none();
    has_ = false;
    py::tuple r = py::make_tuple(src_, dst_, time_, stream_);
    src_ = dst_ = time_ = at::Tensor();
    return r;
  }
  // advance() of the planned batch: commits it when src/dst/time are the planned
  // tensors, feat is None or a contiguous (b, feat_dim) tensor of the ring's dtype
  // on its device, and the current stream is the plan's.  Returns b, or 0 when it
  // did nothing (the caller then takes the general path).
  int64_t commit(const at::Tensor& s, const at::Tensor& d, const at::Tensor& t,
                 const c10::optional<at::Tensor>& feat, int64_t eid_base) {
    if (!matches(s, d, t)) return 0;
    const int64_t b = s.numel();
    const void* fp = nullptr;
    if (feat.has_value()) {
      const at::Tensor& f = *feat;
      if (f.dim() != 2 || f.size(0) != b || f.size(1) != feat_dim_ || f.scalar_type() != feat_dtype_ ||
          f.device() != dev_ || !f.is_contiguous())
        return 0;
      fp = f.data_ptr();
    }
    void* stream = current_stream(dev_.index());
    if (reinterpret_cast<int64_t>(stream) != stream_) return 0;
    has_ = false;
    const int rc = tgx_ring_commit(reinterpret_cast<const tgx_ring*>(ring_), src_.data_ptr<int64_t>(),
                                   dst_.data_ptr<int64_t>(), time_.data_ptr<double>(), fp, b, eid_base,
                                   ws_.data_ptr(), static_cast<size_t>(ws_.numel()),
                                   status_.data_ptr<int32_t>(), stream);
    src_ = dst_ = time_ = at::Tensor();
    check(rc, "tgx_ring_commit");
    return b;
  }
  // drops a pending plan enqueued on `stream` (the caller's current one); false
  // when the plan lives on another stream (the caller orders the streams first)
  bool discard_here(void* stream) {
    if (!has_) return true;
    if (reinterpret_cast<int64_t>(stream) != stream_) return false;
    has_ = false;
    const int rc = tgx_ring_discard(reinterpret_cast<const tgx_ring*>(ring_), src_.data_ptr<int64_t>(),
                                    dst_.data_ptr<int64_t>(), src_.numel(), ws_.data_ptr(),
                                    static_cast<size_t>(ws_.numel()), stream);
    src_ = dst_ = time_ = at::Tensor();
    check(rc, "tgx_ring_discard");
    return true;
  }
  const at::Tensor& ws() const { return ws_; }

 private:
  int64_t ring_;
  at::Tensor status_, ws_;
  int64_t feat_dim_;
  at::ScalarType feat_dtype_;
  at::Device dev_;
  at::Tensor src_, dst_, time_;
  uint32_t ver_[3] = {0, 0, 0};
  int64_t stream_ = 0;
  bool has_ = false;
};

// Generic launch (TemporalGraph.recent, recent_2hop, co_neighbors, the timing
// launches of DataPipeline.launch).  Queries arrive as groups (nodes, times,
// times_per[, valid]) read in place by the kernel.  append_src/dst/time +
// append_ws (all or none): the caller's next ring batch, planned by the same
// launch when plannable() allows.  event_query_groups: as tgx_recent_args, or -1
// for the layout DataPipeline's prepare picks (pair_tail_groups; the group size
// then becomes the pair's times_per sum when the tail applies).
// Returns (planned, tensors): per group ids, times, feats, mask, [te], [eids],
// then co_a, co_c, co_pair with co-occurrence.
py::tuple recent(int64_t ring_addr, int64_t csr_addr, const std::vector<at::Tensor>& gnodes,
                 const std::vector<at::Tensor>& gtimes, const std::vector<int64_t>& gper,
                 const std::vector<c10::optional<at::Tensor>>& gvalid, int64_t k,
                 int64_t feat_dim, at::ScalarType feat_dtype, const c10::optional<at::Tensor>& plan,
                 int64_t plan_mode, int64_t group, int64_t num_groups,
                 int64_t event_query_groups, int64_t d_t,
                 const c10::optional<at::Tensor>& te_w, const c10::optional<at::Tensor>& te_b,
                 double te_bound_w, double te_bound_b,
                 int64_t dt_mode, int64_t co_mode, bool want_eids, const at::Tensor& status,
                 int64_t stream, int64_t ev0, int64_t ev1,
                 const c10::optional<at::Tensor>& append_src,
                 const c10::optional<at::Tensor>& append_dst,
                 const c10::optional<at::Tensor>& append_time,
                 const c10::optional<at::Tensor>& append_ws) {
  const size_t ng = gnodes.size();
  if (ng == 0 || ng > TGX_MAX_QUERY_GROUPS || gtimes.size() != ng || gper.size() != ng ||
      (!gvalid.empty() && gvalid.size() != ng))
    throw std::invalid_argument("recent: 1..4 query groups with matching times");
  const at::Device dev = status.device();
  std::vector<at::Tensor> n(ng), t(ng), v(ng);
  std::vector<int64_t> sizes(ng);
  int64_t Q = 0;
  for (size_t g = 0; g < ng; ++g) {
    // int32 node ids are read as they are (the 2-hop queries are hop-1 ids)
    const at::Tensor fn = flat(gnodes[g]);
    n[g] = as_dev(fn, fn.scalar_type() == at::kInt ? at::kInt : at::kLong, dev);
    t[g] = as_dev(flat(gtimes[g]), at::kDouble, dev);
    if (n[g].numel() != t[g].numel() * gper[g])
      throw std::invalid_argument("recent: query group node/time sizes do not match");
    if (!gvalid.empty() && gvalid[g].has_value()) {
      v[g] = as_dev(flat(*gvalid[g]), at::kBool, dev);
      if (v[g].numel() != n[g].numel())
        throw std::invalid_argument("recent: query group validity size does not match its nodes");
    }
    sizes[g] = n[g].numel();
    Q += sizes[g];
  }
  const Out out(dev, Q, k, feat_dim, feat_dtype, d_t, want_eids, co_mode, num_groups < 0 ? 0 : num_groups);
  tgx_recent_args a{};
  a.num_queries = Q;
  a.k = static_cast<int32_t>(k);
  a.plan = plan.has_value() ? plan->data_ptr<int32_t>() : nullptr;
  a.plan_mode = plan.has_value() ? TGX_PLAN_LIST : static_cast<int32_t>(plan_mode);
  a.group = static_cast<int32_t>(group);
  a.num_groups = num_groups < 0 ? 0 : num_groups;
  if (event_query_groups < 0) {
    int64_t G = 0;
    for (size_t g = 0; g < ng; ++g) G += gper[g];
    event_query_groups = a.plan_mode == TGX_PLAN_EVENTS ? pair_tail_groups(ng, Q, G, k) : 0;
    if (event_query_groups > 0) a.group = static_cast<int32_t>(gper[0] + gper[1]);
  }
  a.event_query_groups = static_cast<int32_t>(event_query_groups);
  out.fill(a);
  a.d_t = static_cast<int32_t>(d_t);
  a.te_w = te_w.has_value() ? te_w->data_ptr<float>() : nullptr;
  a.te_b = te_b.has_value() ? te_b->data_ptr<float>() : nullptr;
  a.te_bound_w = static_cast<float>(te_bound_w);
  a.te_bound_b = static_cast<float>(te_bound_b);
  a.dt_mode = static_cast<int32_t>(dt_mode);
  a.co_mode = static_cast<int32_t>(co_mode);
  a.status = status.data_ptr<int32_t>();
  a.num_query_groups = static_cast<int32_t>(ng);
  for (size_t g = 0; g < ng; ++g) {
    a.query_groups[g].nodes = n[g].data_ptr();
    a.query_groups[g].flags = n[g].scalar_type() == at::kInt ? TGX_QG_NODES_I32 : 0;
    a.query_groups[g].times = t[g].data_ptr<double>();
    a.query_groups[g].count = sizes[g];
    a.query_groups[g].times_per = static_cast<int32_t>(gper[g]);
    a.query_groups[g].valid = v[g].defined() ? reinterpret_cast<const uint8_t*>(v[g].data_ptr<bool>()) : nullptr;
  }
  a.timing_start = reinterpret_cast<void*>(ev0);
  a.timing_stop = reinterpret_cast<void*>(ev1);
  bool planned = false;
  if (append_src.has_value()) {
    if (!append_dst.has_value() || !append_time.has_value() || !append_ws.has_value())
      throw std::invalid_argument("recent: append_src/dst/time/ws come together");
    planned = plannable(*append_src, *append_dst, *append_time, dev);
  }
  if (planned) {
    a.append_src = append_src->data_ptr<int64_t>();
    a.append_dst = append_dst->data_ptr<int64_t>();
    a.append_time = append_time->data_ptr<double>();
    a.append_b = append_src->numel();
    a.append_workspace = append_ws->data_ptr();
    a.append_workspace_bytes = static_cast<size_t>(append_ws->numel());
  }
  if (Q > 0 || a.append_b > 0)
    check(tgx_recent(reinterpret_cast<const tgx_ring*>(ring_addr),
                     reinterpret_cast<const tgx_csr*>(csr_addr), &a,
                     reinterpret_cast<void*>(stream)),
          "tgx_recent");
  std::vector<at::Tensor> res;
  res.reserve(ng * 6 + 3);
  int64_t r0 = 0;
  for (size_t g = 0; g < ng; ++g) {
    out.group(res, r0, sizes[g]);
    r0 += sizes[g];
  }
  if (out.co) out.co_out(res);
  return py::make_tuple(planned, std::move(res));
}

// The 1-hop prepare of one DataPipeline on one graph, configured once: the
// query groups [src, dst, neg (row-major), neg_src] that the spec asks for,
// k, the feature layout, the time encoding and the co-occurrence mode.
// run() takes one batch, launches on the caller's current stream and returns
// the tensors of recent() (without the planned flag), the groups present in
// this batch in that order.
class Prepare {
 public:
  Prepare(int64_t ring_addr, int64_t csr_addr, int64_t groups_mask, int64_t k, int64_t feat_dim,
          at::ScalarType feat_dtype, int64_t d_t, const c10::optional<at::Tensor>& te_w,
          const c10::optional<at::Tensor>& te_b, double te_bound_w, double te_bound_b,
          int64_t dt_mode, int64_t co_mode, bool want_eids,
          int64_t qpw, const at::Tensor& status, std::shared_ptr<PlanSlot> slot)
      : ring_(ring_addr), csr_(csr_addr), mask_(groups_mask), k_(k), feat_dim_(feat_dim),
        feat_dtype_(feat_dtype), d_t_(d_t), te_w_(te_w), te_b_(te_b),
        te_bound_w_(static_cast<float>(te_bound_w)), te_bound_b_(static_cast<float>(te_bound_b)),
        dt_mode_(dt_mode),
        co_mode_(co_mode), want_eids_(want_eids), qpw_(qpw), status_(status),
        dev_(status.device()), slot_(std::move(slot)) {
    if (k < 1 || k > TGX_MAX_K) throw std::invalid_argument("Prepare: k outside [1, TGX_MAX_K]");
    if (co_mode != TGX_CO_NONE && (groups_mask & 3) != 3)
      throw std::invalid_argument("Prepare: co-occurrence needs the src and dst groups");
  }

  // plan: also plan this batch's ring update in the launch (when the graph has a
  // ring and the tensors allow it), for the advance() that follows; a pending
  // plan of an earlier batch on this stream is discarded first.  Returns None,
  // having done nothing, when the plan state needs the caller: an earlier plan
  // pending on another stream, or a plan workspace smaller than this batch needs.
  py::object run(const at::Tensor& src, const at::Tensor& dst, const at::Tensor& time,
                 const c10::optional<at::Tensor>& neg, const c10::optional<at::Tensor>& neg_src,
                 bool plan) const {
    const int64_t b = src.size(0);
    if (dst.size(0) != b || time.size(0) != b)
      throw std::invalid_argument("prepare: src, dst and time must have the same length");
    at::Tensor tt = as_dev(flat(time), at::kDouble, dev_);
    at::Tensor gn[TGX_MAX_QUERY_GROUPS];
    int32_t per[TGX_MAX_QUERY_GROUPS];
    int ng = 0;
    if (mask_ & 1) {
      gn[ng] = as_dev(flat(src), at::kLong, dev_);
      per[ng++] = 1;
    }
    if (mask_ & 2) {
      gn[ng] = as_dev(flat(dst), at::kLong, dev_);
      per[ng++] = 1;
    }
    if ((mask_ & 4) && neg.has_value()) {
      // a (b, n) block is read row-major: n queries per event
      const int64_t p = neg->dim() > 1 ? neg->size(1) : 1;
      if (neg->numel() != b * p) throw std::invalid_argument("prepare: neg must hold b x n nodes");
      gn[ng] = as_dev(flat(*neg), at::kLong, dev_);
      per[ng++] = static_cast<int32_t>(p);
    }
    if ((mask_ & 8) && neg_src.has_value()) {
      if (neg_src->numel() != b) throw std::invalid_argument("prepare: neg_src must hold b nodes");
      gn[ng] = as_dev(flat(*neg_src), at::kLong, dev_);
      per[ng++] = 1;
    }
    int64_t Q = 0;
    int G = 0;
    for (int g = 0; g < ng; ++g) {
      Q += b * per[g];
      G += per[g];
    }
    // event-major groups when the pair must meet in one workgroup
    const bool events = co_mode_ != TGX_CO_NONE;
    const bool tail = events && pair_tail_groups(static_cast<size_t>(ng), Q, G, k_) > 0;
    if (tail) G = per[0] + per[1];
    const Out out(dev_, Q, k_, feat_dim_, feat_dtype_, d_t_, want_eids_, co_mode_, b);
    tgx_recent_args a{};
    a.num_queries = Q;
    a.k = static_cast<int32_t>(k_);
    a.plan_mode = events ? TGX_PLAN_EVENTS : TGX_PLAN_TILES;
    a.group = events ? G : static_cast<int32_t>(qpw_);
    a.num_groups = events ? b : 0;
    a.event_query_groups = tail ? 2 : 0;
    out.fill(a);
    a.d_t = static_cast<int32_t>(d_t_);
    a.te_w = te_w_.has_value() ? te_w_->data_ptr<float>() : nullptr;
    a.te_b = te_b_.has_value() ? te_b_->data_ptr<float>() : nullptr;
    a.te_bound_w = te_bound_w_;
    a.te_bound_b = te_bound_b_;
    a.dt_mode = static_cast<int32_t>(dt_mode_);
    a.co_mode = static_cast<int32_t>(co_mode_);
    a.status = status_.data_ptr<int32_t>();
    a.num_query_groups = ng;
    const double* tp = tt.data_ptr<double>();
    for (int g = 0; g < ng; ++g) {
      a.query_groups[g].nodes = gn[g].data_ptr();
      a.query_groups[g].times = tp;
      a.query_groups[g].count = b * per[g];
      a.query_groups[g].times_per = per[g];
    }
    void* stream = current_stream(dev_.index());
    PlanSlot* slot = plan && ring_ != 0 ? slot_.get() : nullptr;
    const bool planned = slot != nullptr && plannable(src, dst, time, dev_);
    if (slot != nullptr) {
      // an earlier plan nobody advanced is dropped first (it shares the scratch)
      if (slot->pending() && !slot->discard_here(stream)) return py::none();
    }
    if (planned) {
      const at::Tensor& ws = slot->ws();
      if (!ws.defined() || static_cast<size_t>(ws.numel()) < tgx_ring_append_workspace_size(b))
        return py::none();
      a.append_src = src.data_ptr<int64_t>();
      a.append_dst = dst.data_ptr<int64_t>();
      a.append_time = time.data_ptr<double>();
      a.append_b = b;
      a.append_workspace = ws.data_ptr();
      a.append_workspace_bytes = static_cast<size_t>(ws.numel());
    }
    if (Q > 0 || a.append_b > 0)
      check(tgx_recent(reinterpret_cast<const tgx_ring*>(ring_),
                       reinterpret_cast<const tgx_csr*>(csr_), &a, stream),
            "tgx_recent");
    if (planned) slot->record(src, dst, time, reinterpret_cast<int64_t>(stream));
    std::vector<at::Tensor> res;
    res.reserve(ng * 6 + 3);
    int64_t r0 = 0;
    for (int g = 0; g < ng; ++g) {
      out.group(res, r0, b * per[g]);
      r0 += b * per[g];
    }
    if (out.co) out.co_out(res);
    return as_tuple(res);
  }

 private:
  int64_t ring_, csr_, mask_, k_, feat_dim_;
  at::ScalarType feat_dtype_;
  int64_t d_t_;
  c10::optional<at::Tensor> te_w_, te_b_;
  float te_bound_w_, te_bound_b_;
  int64_t dt_mode_, co_mode_;
  bool want_eids_;
  int64_t qpw_;
  at::Tensor status_;
  at::Device dev_;
  std::shared_ptr<PlanSlot> slot_;
};

void ring_append(int64_t ring_addr, const at::Tensor& src, const at::Tensor& dst,
                 const at::Tensor& time, const c10::optional<at::Tensor>& feat,
                 int64_t eid_base, const at::Tensor& workspace, const at::Tensor& status,
                 int64_t stream) {
  const at::Device dev = status.device();
  const int64_t b = src.numel();
  at::Tensor s = as_dev(src, at::kLong, dev);
  at::Tensor d = as_dev(dst, at::kLong, dev);
  at::Tensor t = as_dev(time, at::kDouble, dev);
  if (d.numel() != b || t.numel() != b)
    throw std::invalid_argument("advance: src, dst and time must have the same length");
  check(tgx_ring_append(reinterpret_cast<const tgx_ring*>(ring_addr), s.data_ptr<int64_t>(),
                        d.data_ptr<int64_t>(), t.data_ptr<double>(),
                        feat.has_value() ? feat->data_ptr() : nullptr, b, eid_base,
                        workspace.data_ptr(), static_cast<size_t>(workspace.numel()),
                        status.data_ptr<int32_t>(), reinterpret_cast<void*>(stream)),
        "tgx_ring_append");
}

// the two halves of ring_append (tensors already int64 / float64 / contiguous on
// the device: the caller keeps them alive across both calls)
void ring_plan(int64_t ring_addr, const at::Tensor& src, const at::Tensor& dst,
               const at::Tensor& time, const at::Tensor& workspace, int64_t stream) {
  check(tgx_ring_plan(reinterpret_cast<const tgx_ring*>(ring_addr), src.data_ptr<int64_t>(),
                      dst.data_ptr<int64_t>(), time.data_ptr<double>(), src.numel(),
                      workspace.data_ptr(), static_cast<size_t>(workspace.numel()),
                      reinterpret_cast<void*>(stream)),
        "tgx_ring_plan");
}

void ring_commit(int64_t ring_addr, const at::Tensor& src, const at::Tensor& dst,
                 const at::Tensor& time, const c10::optional<at::Tensor>& feat, int64_t eid_base,
                 const at::Tensor& workspace, const at::Tensor& status, int64_t stream) {
  check(tgx_ring_commit(reinterpret_cast<const tgx_ring*>(ring_addr), src.data_ptr<int64_t>(),
                        dst.data_ptr<int64_t>(), time.data_ptr<double>(),
                        feat.has_value() ? feat->data_ptr() : nullptr, src.numel(), eid_base,
                        workspace.data_ptr(), static_cast<size_t>(workspace.numel()),
                        status.data_ptr<int32_t>(), reinterpret_cast<void*>(stream)),
        "tgx_ring_commit");
}

void ring_discard(int64_t ring_addr, const at::Tensor& src, const at::Tensor& dst,
                  const at::Tensor& workspace, int64_t stream) {
  check(tgx_ring_discard(reinterpret_cast<const tgx_ring*>(ring_addr), src.data_ptr<int64_t>(),
                         dst.data_ptr<int64_t>(), src.numel(), workspace.data_ptr(),
                         static_cast<size_t>(workspace.numel()), reinterpret_cast<void*>(stream)),
        "tgx_ring_discard");
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("recent", &recent, "allocate outputs, launch tgx_recent, return (planned, tensors)");
  py::class_<PlanSlot, std::shared_ptr<PlanSlot>>(m, "PlanSlot")
      .def(py::init<int64_t, const at::Tensor&, int64_t, at::ScalarType>())
      .def("set_workspace", &PlanSlot::set_workspace)
      .def("workspace", &PlanSlot::workspace)
      .def("pending", &PlanSlot::pending)
      .def("stream", &PlanSlot::stream)
      .def("set_stream", &PlanSlot::set_stream)
      .def("record", &PlanSlot::record)
      .def("matches", &PlanSlot::matches)
      .def("take", &PlanSlot::take)
      .def("commit", &PlanSlot::commit, "advance() of the planned batch: b, or 0 (nothing done)");
  py::class_<Prepare>(m, "Prepare")
      .def(py::init<int64_t, int64_t, int64_t, int64_t, int64_t, at::ScalarType, int64_t,
                    const c10::optional<at::Tensor>&, const c10::optional<at::Tensor>&, double,
                    double, int64_t, int64_t, bool, int64_t, const at::Tensor&,
                    std::shared_ptr<PlanSlot>>())
      .def("run", &Prepare::run, "one 1-hop prepare launch: its tensors, or None");
  m.def("ring_append", &ring_append, "launch tgx_ring_append on one batch");
  m.def("ring_plan", &ring_plan, "launch tgx_ring_plan (first half of an append)");
  m.def("ring_commit", &ring_commit, "launch tgx_ring_commit (second half of an append)");
  m.def("ring_discard", &ring_discard, "launch tgx_ring_discard (drop a planned append)");
}
