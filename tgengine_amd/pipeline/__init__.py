"""DataPipeline: the drop-in for tgengine/pipeline/__init__.py:14-219.

``prepare`` keeps the reference's query grouping (``[src, dst, neg (row-major
flatten), neg_src]`` with the matching times, :40-70) and output split, but
runs the whole batch -- gather, feature rows, optional FixedCosineTimeEncoder
and co-occurrence -- in ONE ``tgx_recent`` launch.  With co-occurrence the
launch uses an event-major plan: workgroup p holds event p's queries, src
first and dst second, so the pair meets in one LDS.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch
from torch import Tensor

from tgengine_amd.core import _lib
from tgengine_amd.core.batch import NeighborData, PreparedBatch, RawBatch
from tgengine_amd.core.gather_spec import GatherSpec
from tgengine_amd.core.temporal_graph import TemporalGraph

_DT_MODES = {"dygformer": _lib.TGX_DT_DYGFORMER, "tgn": _lib.TGX_DT_TGN}
_CO_MODES = {"freq": _lib.TGX_CO_FREQ, "dygformer": _lib.TGX_CO_DYGFORMER}
_PLAN_CACHE_ENTRIES = 64  # query plans and (plan, group) pairs kept per pipeline


def cosine_time_weights(d_t: int) -> np.ndarray:
    """w = 1/10**linspace(0, 9, d_t) in fp32 (tgengine/nn/time_encoding.py:49)."""
    return (1.0 / (10 ** np.linspace(0, 9, d_t, dtype=np.float32))).astype(np.float32)


def event_plan(b: int, groups: list) -> np.ndarray:
    """Event-major plan: row p lists event p's query indices in ``groups`` order.

    ``groups`` is [(offset, per_event)] for each query group in the flattened
    query list; group g of event p owns indices offset + p*per_event + j.
    """
    cols = []
    p = np.arange(b, dtype=np.int64)
    for off, per in groups:
        for j in range(per):
            cols.append(off + p * per + j)
    return np.stack(cols, 1).astype(np.int32).reshape(-1)


class DataPipeline:
    """``time_encoder``: optional module with a ``linear`` Linear(1, d_t) whose
    weight/bias replace the fixed cosine frequencies.  ``queries_per_workgroup``:
    queries one workgroup (one wavefront each) gathers when no co-occurrence pair
    has to share a workgroup."""

    def __init__(self, spec: GatherSpec, graph: TemporalGraph, time_encoder=None,
                 queries_per_workgroup: int = 4):
        if not 1 <= queries_per_workgroup <= _lib.TGX_MAX_GROUP:
            raise ValueError(f"queries_per_workgroup must be in [1, {_lib.TGX_MAX_GROUP}]")
        self.spec = spec
        self.graph = graph
        self.time_encoder = time_encoder
        self.queries_per_workgroup = int(queries_per_workgroup)
        # plan the ring update of each prepared batch inside its gather launch
        # (the plan writes only the ring's scratch); the following advance() of
        # the same tensors then makes a single commit launch
        self.plan_updates = True
        self._plans: dict = {}
        self._te: dict = {}

    # -- cached device constants ------------------------------------------
    def _te_params(self, d_t: int):
        """(w, b) device tensors; b is None for a zero bias."""
        enc = self.time_encoder
        if enc is not None:
            w = enc.linear.weight.detach().reshape(-1).to(self.graph.device, torch.float32).contiguous()
            bias = enc.linear.bias
            b = None
            if bias is not None and bool(torch.any(bias.detach() != 0)):
                b = bias.detach().to(self.graph.device, torch.float32).contiguous()
            if w.numel() != d_t:
                raise ValueError(f"time encoder has {w.numel()} frequencies, spec asks for {d_t}")
            return w, b
        t = self._te.get(d_t)
        if t is None:
            t = torch.from_numpy(cosine_time_weights(d_t)).to(self.graph.device)
            self._te[d_t] = t
        return t, None

    def _event_plan(self, b: int, per_event: list) -> tuple:
        """(plan, queries per event) of the event-major grouping [src p, dst p, its
        negatives, neg_src p] of a batch of b events, cached per shape."""
        key = (b, *per_event)
        hit = self._plans.get(key)
        if hit is not None:
            return hit
        offs, off = [], 0
        for per in per_event:
            offs.append((off, per))
            off += b * per
        G = sum(per_event)
        if G > _lib.TGX_MAX_GROUP:
            raise ValueError(f"{G} queries per event exceed the fused group limit {_lib.TGX_MAX_GROUP}")
        hit = (self._plan(("ev", b, tuple(per_event)), b, offs), G)
        self._remember(key, hit)
        return hit

    def _plan(self, key, b: int, groups: list) -> Tensor:
        t = self._plans.get(key)
        if t is None:
            t = torch.from_numpy(event_plan(b, groups)).to(self.graph.device)
            self._remember(key, t)
        return t

    def _remember(self, key, value) -> None:
        """Caches per batch shape, dropping the oldest shapes beyond a bound so a
        stream of many batch sizes (time-window batching) keeps the cache small.
        A dropped plan may still be read by a queued launch on another stream, so
        the device drains first (rare: only past the bound)."""
        if len(self._plans) >= _PLAN_CACHE_ENTRIES:
            torch.cuda.synchronize(self.graph.device)
            while len(self._plans) >= _PLAN_CACHE_ENTRIES:
                del self._plans[next(iter(self._plans))]
        self._plans[key] = value

    # -- prepare -------------------------------------------------------------
    def _query_groups(self, raw_batch: RawBatch):
        """Query groups in the reference order [src, dst, neg (row-major), neg_src],
        read in place by the kernel: names, (nodes, times, negatives per event),
        sizes and negatives per event (pipeline/__init__.py:40-70)."""
        fn = self.spec.neighbors.for_nodes
        b = raw_batch.src.shape[0]
        names, qgroups, sizes, per_event = [], [], [], []
        if "src" in fn:
            names.append("src"); qgroups.append((raw_batch.src, raw_batch.time, 1))
            sizes.append(b); per_event.append(1)
        if "dst" in fn:
            names.append("dst"); qgroups.append((raw_batch.dst, raw_batch.time, 1))
            sizes.append(b); per_event.append(1)
        if "neg" in fn and raw_batch.neg is not None:
            neg = raw_batch.neg  # a (b, n) block is read row-major (the host glue flattens it)
            per = neg.shape[1] if neg.ndim > 1 else 1
            names.append("neg"); qgroups.append((neg, raw_batch.time, per))
            sizes.append(neg.numel()); per_event.append(per)
        if "neg" in fn and raw_batch.neg_src is not None:
            names.append("neg_src"); qgroups.append((raw_batch.neg_src, raw_batch.time, 1))
            sizes.append(b); per_event.append(1)
        return names, qgroups, sizes, per_event

    def launch_args(self, raw_batch: RawBatch) -> tuple:
        """(d_t, te_w, te_b, dt_mode, co_mode) of the fused launch for this spec."""
        spec = self.spec
        fn = spec.neighbors.for_nodes
        want_co = spec.co_occurrence and "src" in fn and "dst" in fn
        co_mode = _CO_MODES[spec.co_occurrence_mode] if want_co else _lib.TGX_CO_NONE
        d_t = int(spec.time_encoding)
        te_w = te_b = None
        if d_t > 0:
            te_w, te_b = self._te_params(d_t)
        return d_t, te_w, te_b, _DT_MODES[spec.dt_mode], co_mode

    def launch(self, raw_batch: RawBatch, args: Optional[tuple] = None) -> dict:
        """The one fused tgx_recent launch of ``prepare`` (1-hop), returning its raw
        output views (lists per query group) without building a PreparedBatch;
        for timing loops that must not be host-bound."""
        names, qgroups, _, per_event = self._query_groups(raw_batch)
        d_t, te_w, te_b, dt_mode, co_mode = args if args is not None else self.launch_args(raw_batch)
        if "src" not in names or "dst" not in names:
            co_mode = _lib.TGX_CO_NONE
        return self._fused(qgroups, self.spec.neighbors.k, raw_batch.src.shape[0], per_event, d_t,
                           te_w, te_b, dt_mode, co_mode)

    def prepare(self, raw_batch: RawBatch) -> PreparedBatch:
        spec = self.spec
        if spec.neighbors.k2 == 0:
            return self._prepare_1hop(raw_batch)
        k, k2 = spec.neighbors.k, spec.neighbors.k2
        device = raw_batch.device
        b = raw_batch.src.shape[0]
        names, qgroups, sizes, per_event = self._query_groups(raw_batch)
        append = (raw_batch.src, raw_batch.dst, raw_batch.time) if self.plan_updates else None

        if spec.edge_ids and not self.graph.track_edge_ids:
            raise ValueError("GatherSpec.edge_ids needs a TemporalGraph built with track_edge_ids=True")
        want_co = spec.co_occurrence and "src" in names and "dst" in names
        co_mode = _CO_MODES[spec.co_occurrence_mode] if want_co else _lib.TGX_CO_NONE
        d_t = int(spec.time_encoding)
        te_w = te_b = None
        if d_t > 0:
            te_w, te_b = self._te_params(d_t)
        dt_mode = _DT_MODES[spec.dt_mode]

        if k2 > 0:
            if append is not None:  # several launches here: the plan gets its own
                self.graph.plan_append(*append)
            all_nodes = torch.cat([g[0].reshape(-1) for g in qgroups])
            all_times = torch.cat([g[1].repeat_interleave(g[2]) if g[2] > 1 else g[1]
                                   for g in qgroups])
            hop = self.graph.recent_2hop(all_nodes, all_times, k, k2)

            def split(t):
                return None if t is None else torch.split_with_sizes(t, sizes, dim=0)

            out = {"ids": split(hop.neighbor_ids), "times": split(hop.timestamps),
                   "feats": split(hop.edge_feats), "mask": split(hop.mask),
                   "eids": split(hop.edge_ids)}
            extra = {"hop2_ids": hop.hop2_ids, "hop2_times": hop.hop2_times,
                     "hop2_feats": hop.hop2_feats, "hop2_mask": hop.hop2_mask}
            if d_t > 0 or want_co:
                o2 = self._fused(qgroups, k, b, per_event, d_t, te_w, te_b, dt_mode, co_mode)
                out.update({kk: o2[kk] for kk in ("te", "co_a", "co_c", "co_pair") if kk in o2})
        else:
            out = self._fused(qgroups, k, b, per_event, d_t, te_w, te_b, dt_mode, co_mode,
                              append=append)
            extra = {}

        parts = {kk: out.get(kk) for kk in ("ids", "times", "feats", "mask", "te", "eids")}
        hparts = {kk: torch.split_with_sizes(v, sizes, dim=0) for kk, v in extra.items()}
        nbrs = {}
        for i, name in enumerate(names):
            nd = NeighborData(parts["ids"][i], parts["times"][i], parts["feats"][i], parts["mask"][i])
            if parts["te"] is not None:
                nd.time_enc = parts["te"][i]
            if parts["eids"] is not None:
                nd.edge_ids = parts["eids"][i]
            for kk, v in hparts.items():
                setattr(nd, kk, v[i])
            nbrs[name] = nd

        co_occur = co_freq = None
        if spec.co_occurrence:
            if want_co:
                co_occur = out["co_pair"]
                co_freq = (out["co_a"], out["co_c"])
            else:
                co_occur = self.graph.co_neighbors(raw_batch.src, raw_batch.dst, raw_batch.time, k=k)

        return PreparedBatch(
            src=raw_batch.src, dst=raw_batch.dst,
            neg=raw_batch.neg if raw_batch.neg is not None else torch.empty(0, device=device),
            time=raw_batch.time,
            src_neighbors=nbrs.get("src"), dst_neighbors=nbrs.get("dst"),
            neg_neighbors=nbrs.get("neg"), neg_src_neighbors=nbrs.get("neg_src"),
            neg_src=raw_batch.neg_src, co_occurrence=co_occur,
            node_labels=raw_batch.node_labels, edge_labels=raw_batch.edge_labels,
            node_feat=raw_batch.node_feat, co_occurrence_freq=co_freq)

    def _prepare_1hop(self, raw_batch: RawBatch) -> PreparedBatch:
        """prepare() of a 1-hop spec: one launch (gather, time encoding,
        co-occurrence and the plan of this batch's ring update), its per-group
        views put straight into the NeighborData of each group."""
        spec = self.spec
        g = self.graph
        names, qgroups, _, per_event = self._query_groups(raw_batch)
        if spec.edge_ids and not g.track_edge_ids:
            raise ValueError("GatherSpec.edge_ids needs a TemporalGraph built with track_edge_ids=True")
        want_co = spec.co_occurrence and "src" in names and "dst" in names
        co_mode = _CO_MODES[spec.co_occurrence_mode] if want_co else _lib.TGX_CO_NONE
        d_t = int(spec.time_encoding)
        te_w = te_b = None
        if d_t > 0:
            te_w, te_b = self._te_params(d_t)
        src = raw_batch.src
        append = (src, raw_batch.dst, raw_batch.time) if self.plan_updates else None
        k = spec.neighbors.k
        b = src.shape[0]
        if co_mode != _lib.TGX_CO_NONE:
            plan, G = self._event_plan(b, per_event)
            res = g._gather(qgroups, k, plan, G, b, d_t, te_w, te_b, _DT_MODES[spec.dt_mode],
                            co_mode, spec.edge_ids, append)
        else:
            res = g._gather(qgroups, k, None, self.queries_per_workgroup, None, d_t, te_w, te_b,
                            _DT_MODES[spec.dt_mode], co_mode, spec.edge_ids, append)
        ids, tms, fts, msk, eids, te = res[0], res[1], res[2], res[3], res[4], res[5]
        nbrs = {}
        for i, name in enumerate(names):
            nd = NeighborData(ids[i], tms[i], fts[i], msk[i])
            if te:
                nd.time_enc = te[i]
            if eids:
                nd.edge_ids = eids[i]
            nbrs[name] = nd
        co_occur = co_freq = None
        if spec.co_occurrence:
            if want_co:
                co_a, co_c, co_occur = res[6]
                co_freq = (co_a, co_c)
            else:
                co_occur = g.co_neighbors(src, raw_batch.dst, raw_batch.time, k=k)
        neg = raw_batch.neg
        return PreparedBatch(
            src=src, dst=raw_batch.dst,
            neg=neg if neg is not None else torch.empty(0, device=src.device),
            time=raw_batch.time,
            src_neighbors=nbrs.get("src"), dst_neighbors=nbrs.get("dst"),
            neg_neighbors=nbrs.get("neg"), neg_src_neighbors=nbrs.get("neg_src"),
            neg_src=raw_batch.neg_src, co_occurrence=co_occur,
            node_labels=raw_batch.node_labels, edge_labels=raw_batch.edge_labels,
            node_feat=raw_batch.node_feat, co_occurrence_freq=co_freq)

    def _fused(self, qgroups, k, b, per_event, d_t, te_w, te_b, dt_mode, co_mode,
               append=None) -> dict:
        g = self.graph
        if co_mode != _lib.TGX_CO_NONE:
            # event-major groups: event p -> [src p, dst p, its negatives, neg_src p]
            offs, off = [], 0
            for per in per_event:
                offs.append((off, per))
                off += b * per
            G = sum(per_event)
            if G > _lib.TGX_MAX_GROUP:
                raise ValueError(f"{G} queries per event exceed the fused group limit {_lib.TGX_MAX_GROUP}")
            plan = self._plan(("ev", b, tuple(per_event)), b, offs)
            return g._query(None, None, k, groups=qgroups, plan=plan, group=G, num_groups=b,
                            d_t=d_t, te_w=te_w, te_b=te_b, dt_mode=dt_mode, co_mode=co_mode,
                            want_eids=self.spec.edge_ids, append=append)
        return g._query(None, None, k, groups=qgroups, group=self.queries_per_workgroup,
                        d_t=d_t, te_w=te_w, te_b=te_b, dt_mode=dt_mode,
                        want_eids=self.spec.edge_ids, append=append)

    @staticmethod
    def _co_occur_from_neighbors(src_nbrs: NeighborData, dst_nbrs: NeighborData) -> Tensor:
        """(B,) float shared-neighbour count from already-gathered neighbours
        (reference pipeline/__init__.py:206-219), computed by tgx_co_occurrence."""
        a = src_nbrs.neighbor_ids.contiguous()
        c = dst_nbrs.neighbor_ids.contiguous()
        P, K = a.shape
        dev = a.device
        a_cnt = torch.empty((P, K, 2), dtype=torch.int32, device=dev)
        c_cnt = torch.empty((P, K, 2), dtype=torch.int32, device=dev)
        pair = torch.empty((P,), dtype=torch.float32, device=dev)
        if P and K:
            rc = _lib.lib().tgx_co_occurrence(a.data_ptr(), c.data_ptr(), P, K, a_cnt.data_ptr(),
                                              c_cnt.data_ptr(), pair.data_ptr(),
                                              torch.cuda.current_stream(dev).cuda_stream)
            _lib.check(rc, "tgx_co_occurrence")
        else:
            pair.zero_()
        return pair


from tgengine_amd.pipeline.async_pipeline import AsyncDataPipeline  # noqa: E402

__all__ = ["DataPipeline", "AsyncDataPipeline", "cosine_time_weights", "event_plan"]
