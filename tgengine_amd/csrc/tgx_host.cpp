// Host glue of the Python API (torch extension module `tgengine_amd._tgx_host`).
//
// One call per TemporalGraph.recent / DataPipeline.prepare / advance: it checks
// the inputs, allocates the outputs from the caching allocator, fills the C-ABI
// argument block, launches through libtgx and returns the per-group views.  This
// keeps the per-batch host cost to a few microseconds; all device work is in
// libtgx (include/tgx.h), which never sees a torch type.
#include <torch/extension.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "tgx.h"

namespace {

void check(int rc, const char* what) {
  if (rc != TGX_OK) throw std::runtime_error(std::string(what) + " failed: " + tgx_last_error());
}

at::Tensor as_dev(const at::Tensor& t, at::ScalarType dt, const at::Device& dev) {
  if (t.scalar_type() == dt && t.device() == dev && t.is_contiguous()) return t;
  return t.to(dev, dt).contiguous();
}

int64_t ptr(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? reinterpret_cast<int64_t>(t->data_ptr()) : 0;
}

// 1-D view of t (t itself when it already is 1-D)
at::Tensor flat(const at::Tensor& t) { return t.dim() == 1 ? t : t.reshape({-1}); }

// a contiguous `st` tensor of shape `sizes` at byte offset `byte_off` of base's
// storage (a multiple of the element size), built directly like split_rows' blocks
at::Tensor typed_block(const at::Tensor& base, at::ScalarType st, int64_t byte_off,
                       at::IntArrayRef sizes) {
  const caffe2::TypeMeta dt = c10::scalarTypeToTypeMeta(st);
  auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(base.storage()), base.key_set(), dt);
  impl->set_sizes_contiguous(sizes);
  impl->set_storage_offset(byte_off / static_cast<int64_t>(dt.itemsize()));
  return at::Tensor(std::move(impl));
}

// x split along dim 0 into consecutive blocks of sizes[g] rows: tensors built
// directly on x's storage (no dispatcher round trip per block, about four times
// cheaper than split_with_sizes; the blocks are plain tensors sharing x's
// memory, not autograd views of x)
std::vector<at::Tensor> split_rows(const at::Tensor& x, const std::vector<int64_t>& sizes) {
  if (sizes.size() == 1) return {x};
  std::vector<at::Tensor> out;
  out.reserve(sizes.size());
  const c10::Storage& st = x.storage();
  const c10::DispatchKeySet ks = x.key_set();
  const caffe2::TypeMeta dt = x.dtype();
  std::vector<int64_t> sz(x.sizes().begin(), x.sizes().end());
  const at::IntArrayRef strides = x.strides();
  int64_t off = x.storage_offset();
  for (int64_t s : sizes) {
    sz[0] = s;
    auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(st), ks, dt);
    impl->set_sizes_and_strides(sz, strides, off);
    out.emplace_back(std::move(impl));
    off += s * strides[0];
  }
  return out;
}

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

// Queries arrive as groups (nodes, times, times_per) read in place by the kernel.
// append_src/dst/time + append_ws (all or none): the caller's next ring batch,
// planned by the same launch when plannable() allows.
// Returns [ids, times, feats, mask(bool), eids|None-placeholder, te|placeholder,
//          co_a, co_c, co_pair, planned] as lists of per-group views (co_*
// unsplit); planned holds one tensor when the batch was planned, else nothing.
std::vector<std::vector<at::Tensor>> recent(
    int64_t ring_addr, int64_t csr_addr, const std::vector<at::Tensor>& gnodes,
    const std::vector<at::Tensor>& gtimes, const std::vector<int64_t>& gper,
    const std::vector<c10::optional<at::Tensor>>& gvalid, int64_t k,
    int64_t feat_dim, at::ScalarType feat_dtype, const c10::optional<at::Tensor>& plan,
    int64_t group, int64_t num_groups, int64_t d_t, const c10::optional<at::Tensor>& te_w,
    const c10::optional<at::Tensor>& te_b, int64_t dt_mode, int64_t co_mode, bool want_eids,
    const at::Tensor& status, int64_t stream, int64_t ev0, int64_t ev1,
    const c10::optional<at::Tensor>& append_src, const c10::optional<at::Tensor>& append_dst,
    const c10::optional<at::Tensor>& append_time, const c10::optional<at::Tensor>& append_ws) {
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
  if (num_groups < 0) num_groups = (Q + group - 1) / group;
  // The small outputs (times, edge ids, ids, co-occurrence, mask) share one
  // allocation, laid out so every offset is a multiple of its element size; the
  // feature rows and encodings, which dominate the bytes, get their own.
  const int64_t QK = Q * k;
  const int64_t L = co_mode == TGX_CO_FREQ ? k : k + 1;
  const int64_t nco = co_mode != TGX_CO_NONE ? num_groups * L * 2 : 0;
  const int64_t o_eids = QK * 8;
  const int64_t o_ids = o_eids + (want_eids ? QK * 8 : 0);
  const int64_t o_coa = o_ids + QK * 4;
  const int64_t o_coc = o_coa + nco * 4;
  const int64_t o_cop = o_coc + nco * 4;
  const int64_t o_msk = o_cop + (co_mode != TGX_CO_NONE ? num_groups * 4 : 0);
  at::Tensor small = at::empty({o_msk + QK}, at::TensorOptions().device(dev).dtype(at::kByte));
  at::Tensor tms = typed_block(small, at::kDouble, 0, {Q, k});
  at::Tensor ids = typed_block(small, at::kInt, o_ids, {Q, k});
  at::Tensor msk = typed_block(small, at::kBool, o_msk, {Q, k});
  at::Tensor fts = at::empty({Q, k, feat_dim}, at::TensorOptions().device(dev).dtype(feat_dtype));
  c10::optional<at::Tensor> eids, te, co_a, co_c, co_pair;
  if (want_eids) eids = typed_block(small, at::kLong, o_eids, {Q, k});
  if (d_t > 0) te = at::empty({Q, k, d_t}, at::TensorOptions().device(dev).dtype(at::kFloat));
  if (co_mode != TGX_CO_NONE) {
    co_a = typed_block(small, at::kInt, o_coa, {num_groups, L, 2});
    co_c = typed_block(small, at::kInt, o_coc, {num_groups, L, 2});
    co_pair = typed_block(small, at::kFloat, o_cop, {num_groups});
  }
  tgx_recent_args a{};
  a.num_queries = Q;
  a.k = static_cast<int32_t>(k);
  a.plan = plan.has_value() ? plan->data_ptr<int32_t>() : nullptr;
  a.group = static_cast<int32_t>(group);
  a.num_groups = num_groups;
  a.out_ids = ids.data_ptr<int32_t>();
  a.out_times = tms.data_ptr<double>();
  a.out_feats = fts.data_ptr();
  a.out_mask = reinterpret_cast<uint8_t*>(msk.data_ptr<bool>());
  a.out_eids = eids.has_value() ? eids->data_ptr<int64_t>() : nullptr;
  a.d_t = static_cast<int32_t>(d_t);
  a.te_w = te_w.has_value() ? te_w->data_ptr<float>() : nullptr;
  a.te_b = te_b.has_value() ? te_b->data_ptr<float>() : nullptr;
  a.dt_mode = static_cast<int32_t>(dt_mode);
  a.out_te = te.has_value() ? te->data_ptr<float>() : nullptr;
  a.co_mode = static_cast<int32_t>(co_mode);
  a.co_a = co_a.has_value() ? co_a->data_ptr<int32_t>() : nullptr;
  a.co_c = co_c.has_value() ? co_c->data_ptr<int32_t>() : nullptr;
  a.co_pair = co_pair.has_value() ? co_pair->data_ptr<float>() : nullptr;
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
  std::vector<std::vector<at::Tensor>> out;
  out.reserve(8);
  auto split = [&](const at::Tensor& x) { return split_rows(x, sizes); };
  out.push_back(split(ids));
  out.push_back(split(tms));
  out.push_back(split(fts));
  out.push_back(split(msk));
  out.push_back(eids.has_value() ? split(*eids) : std::vector<at::Tensor>{});
  out.push_back(te.has_value() ? split(*te) : std::vector<at::Tensor>{});
  if (co_mode != TGX_CO_NONE) out.push_back({*co_a, *co_c, *co_pair});
  else out.push_back({});
  if (planned) out.push_back({*append_src});
  else out.push_back({});
  return out;
}

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
  m.def("recent", &recent, "allocate outputs, launch tgx_recent, return per-group views");
  m.def("ring_append", &ring_append, "launch tgx_ring_append on one batch");
  m.def("ring_plan", &ring_plan, "launch tgx_ring_plan (first half of an append)");
  m.def("ring_commit", &ring_commit, "launch tgx_ring_commit (second half of an append)");
  m.def("ring_discard", &ring_discard, "launch tgx_ring_discard (drop a planned append)");
}
