"""DataPipeline: the drop-in for tgengine/pipeline/__init__.py:14-219.

``prepare`` keeps the reference's query grouping (``[src, dst, neg (row-major
flatten), neg_src]`` with the matching times, :40-70) and output split, but
runs the whole batch -- gather, feature rows, optional FixedCosineTimeEncoder
and co-occurrence -- in ONE ``tgx_recent`` launch.  With co-occurrence the
launch uses the event-major plan (computed in the kernel from the query
groups): workgroup p holds event p's queries, src first and dst second, so the
pair meets in one LDS; a launch of at most 4,096 queries puts only that pair in
the event's workgroup and tiles the negatives after them.

The per-batch host path is one call into the extension's ``Prepare`` context,
configured once per (graph arrays, spec) and rebuilt when either changes.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch
from torch import Tensor

from tgengine_amd.core import _lib
from tgengine_amd.core.batch import NeighborData, PreparedBatch, RawBatch
from tgengine_amd.core.gather_spec import GatherSpec
from tgengine_amd.core.temporal_graph import TemporalGraph, _host

_DT_MODES = {"dygformer": _lib.TGX_DT_DYGFORMER, "tgn": _lib.TGX_DT_TGN}
_CO_MODES = {"freq": _lib.TGX_CO_FREQ, "dygformer": _lib.TGX_CO_DYGFORMER}
_GROUP_BITS = {"src": 1, "dst": 2, "neg": 4}


def cosine_time_weights(d_t: int) -> np.ndarray:
    """w = 1/10**linspace(0, 9, d_t) in fp32 (tgengine/nn/time_encoding.py:49)."""
    return (1.0 / (10 ** np.linspace(0, 9, d_t, dtype=np.float32))).astype(np.float32)


def event_plan(b: int, groups: list) -> np.ndarray:
    """The event-major query order (TGX_PLAN_EVENTS) as an explicit plan: row p
    lists event p's query indices in ``groups`` order.

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
    weight/bias replace the fixed cosine frequencies (read in place at every
    launch, so updates to them apply).  ``queries_per_workgroup``: queries one
    workgroup gathers when no co-occurrence pair has to share a workgroup and no
    query is shared by several wavefronts (a small launch gives each such query
    a workgroup of its own)."""

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
        self._te: dict = {}
        self._ctx = None  # (key, extension Prepare context, fields per group)

    # -- cached device constants ------------------------------------------
    def _te_params(self, d_t: int):
        """(w, b, bounds): device tensors, b None for no bias, and the upper
        bounds (max|w|, max|b|) that let the kernel skip the cosine's large-argument
        reduction, (0, 0) when unknown.  With an encoder module its parameters are
        passed as they are when already contiguous float32 on the graph's device
        (a zero bias gives the same encodings as none); their bounds are left
        unknown, since reading them would wait for the device."""
        enc = self.time_encoder
        if enc is not None:
            dev = self.graph.device
            w = enc.linear.weight.detach().reshape(-1).to(dev, torch.float32).contiguous()
            bias = enc.linear.bias
            b = None if bias is None else bias.detach().to(dev, torch.float32).contiguous()
            if w.numel() != d_t:
                raise ValueError(f"time encoder has {w.numel()} frequencies, spec asks for {d_t}")
            return w, b, (0.0, 0.0)
        t = self._te.get(d_t)
        if t is None:
            wn = cosine_time_weights(d_t)
            t = (torch.from_numpy(wn).to(self.graph.device), (float(np.abs(wn).max()), 0.0))
            self._te[d_t] = t
        return t[0], None, t[1]

    def _context(self):
        """The extension's Prepare context for the current graph arrays and spec."""
        spec = self.spec
        g = self.graph
        nb = spec.neighbors
        key = (g._gen, nb.k, nb.for_nodes, spec.time_encoding, spec.dt_mode, spec.co_occurrence,
               spec.co_occurrence_mode, spec.edge_ids, self.queries_per_workgroup,
               id(self.time_encoder))
        ctx = self._ctx
        if ctx is not None and ctx[0] == key and self.time_encoder is None:
            return ctx
        fn = nb.for_nodes
        mask = 0
        for name, bit in _GROUP_BITS.items():
            if name in fn:
                mask |= bit
        if "neg" in fn:
            mask |= 8  # neg_src rides with the negatives, as in the reference
        if spec.edge_ids and not g.track_edge_ids:
            raise ValueError("GatherSpec.edge_ids needs a TemporalGraph built with track_edge_ids=True")
        want_co = spec.co_occurrence and "src" in fn and "dst" in fn
        co_mode = _CO_MODES[spec.co_occurrence_mode] if want_co else _lib.TGX_CO_NONE
        d_t = int(spec.time_encoding)
        te_w = te_b = None
        te_bounds = (0.0, 0.0)
        if d_t > 0:
            te_w, te_b, te_bounds = self._te_params(d_t)
        ring, csr = g._structs()
        prep = _host().Prepare(ring, csr, mask, int(nb.k), g.edge_feat_dim, g.feat_dtype, d_t, te_w,
                               te_b, te_bounds[0], te_bounds[1], _DT_MODES[spec.dt_mode], co_mode,
                               bool(spec.edge_ids),
                               self.queries_per_workgroup, g._status, g._slot)
        self._ctx = (key, prep, 4 + (d_t > 0) + bool(spec.edge_ids), d_t > 0, bool(spec.edge_ids),
                     mask, want_co)
        return self._ctx

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
        """(d_t, te_w, te_b, te_bounds, dt_mode, co_mode) of the fused launch for
        this spec."""
        spec = self.spec
        fn = spec.neighbors.for_nodes
        want_co = spec.co_occurrence and "src" in fn and "dst" in fn
        co_mode = _CO_MODES[spec.co_occurrence_mode] if want_co else _lib.TGX_CO_NONE
        d_t = int(spec.time_encoding)
        te_w = te_b = None
        te_bounds = (0.0, 0.0)
        if d_t > 0:
            te_w, te_b, te_bounds = self._te_params(d_t)
        return d_t, te_w, te_b, te_bounds, _DT_MODES[spec.dt_mode], co_mode

    def launch(self, raw_batch: RawBatch, args: Optional[tuple] = None) -> dict:
        """The one fused tgx_recent launch of ``prepare`` (1-hop) without its ring
        plan, returning its raw output tensors (lists per query group) without
        building a PreparedBatch; for timing loops and graph capture."""
        names, qgroups, _, per_event = self._query_groups(raw_batch)
        d_t, te_w, te_b, te_bounds, dt_mode, co_mode = (args if args is not None
                                                         else self.launch_args(raw_batch))
        if "src" not in names or "dst" not in names:
            co_mode = _lib.TGX_CO_NONE
        return self._fused(qgroups, self.spec.neighbors.k, raw_batch.src.shape[0], per_event, d_t,
                           te_w, te_b, te_bounds, dt_mode, co_mode)

    def prepare(self, raw_batch: RawBatch) -> PreparedBatch:
        if self.spec.neighbors.k2 == 0:
            return self._prepare_1hop(raw_batch)
        return self._prepare_2hop(raw_batch)

    def _prepare_1hop(self, raw_batch: RawBatch) -> PreparedBatch:
        """prepare() of a 1-hop spec: one launch (gather, time encoding,
        co-occurrence and the plan of this batch's ring update) through the
        extension's Prepare context; its per-group tensors go straight into the
        NeighborData of each group."""
        g = self.graph
        if not g._frozen:
            g.freeze_csr()
        _, prep, nf, has_te, has_eids, mask, want_co = self._context()
        src, dst, tm = raw_batch.src, raw_batch.dst, raw_batch.time
        neg, neg_src = raw_batch.neg, raw_batch.neg_src
        res = prep.run(src, dst, tm, neg, neg_src, self.plan_updates)
        if res is None:  # the plan state needs settling first
            res = g._prepare(prep, src, dst, tm, neg, neg_src, self.plan_updates)
        nbrs = [None, None, None, None]
        i = 0
        for slot, bit, present in ((0, 1, True), (1, 2, True), (2, 4, neg is not None),
                                   (3, 8, neg_src is not None)):
            if mask & bit and present:
                nbrs[slot] = NeighborData(res[i], res[i + 1], res[i + 2], res[i + 3], None, None, None,
                                          None, res[i + 4] if has_te else None,
                                          res[i + nf - 1] if has_eids else None)
                i += nf
        co_occur = co_freq = None
        if self.spec.co_occurrence:
            if want_co:
                co_freq = (res[i], res[i + 1])
                co_occur = res[i + 2]
            else:
                co_occur = g.co_neighbors(src, dst, tm, k=self.spec.neighbors.k)
        return PreparedBatch(
            src, dst, neg if neg is not None else torch.empty(0, device=src.device), tm,
            nbrs[0], nbrs[1], nbrs[2], nbrs[3], neg_src, co_occur, None,
            raw_batch.node_labels, raw_batch.edge_labels, raw_batch.node_feat, co_freq)

    def _prepare_2hop(self, raw_batch: RawBatch) -> PreparedBatch:
        """prepare() of a 2-hop spec: the reference's two-launch shape (hop 1 over
        the concatenated queries, then one query per hop-1 slot), plus the fused
        launch for time encodings / co-occurrence when the spec asks for them.
        The ring update of this batch is planned by a launch of its own."""
        spec = self.spec
        k, k2 = spec.neighbors.k, spec.neighbors.k2
        device = raw_batch.device
        b = raw_batch.src.shape[0]
        names, qgroups, sizes, per_event = self._query_groups(raw_batch)
        if spec.edge_ids and not self.graph.track_edge_ids:
            raise ValueError("GatherSpec.edge_ids needs a TemporalGraph built with track_edge_ids=True")
        d_t, te_w, te_b, te_bounds, dt_mode, co_mode = self.launch_args(raw_batch)
        want_co = co_mode != _lib.TGX_CO_NONE
        if self.plan_updates:
            self.graph.plan_append(raw_batch.src, raw_batch.dst, raw_batch.time)
        all_nodes = torch.cat([q[0].reshape(-1) for q in qgroups])
        all_times = torch.cat([q[1].repeat_interleave(q[2]) if q[2] > 1 else q[1] for q in qgroups])
        hop = self.graph.recent_2hop(all_nodes, all_times, k, k2)

        def split(t):
            return None if t is None else torch.split_with_sizes(t, sizes, dim=0)

        parts = {"ids": split(hop.neighbor_ids), "times": split(hop.timestamps),
                 "feats": split(hop.edge_feats), "mask": split(hop.mask), "eids": split(hop.edge_ids),
                 "te": None}
        out = {}
        if d_t > 0 or want_co:
            out = self._fused(qgroups, k, b, per_event, d_t, te_w, te_b, te_bounds, dt_mode, co_mode)
            parts["te"] = out.get("te")
        hparts = {kk: torch.split_with_sizes(v, sizes, dim=0)
                  for kk, v in (("hop2_ids", hop.hop2_ids), ("hop2_times", hop.hop2_times),
                                ("hop2_feats", hop.hop2_feats), ("hop2_mask", hop.hop2_mask))}
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

    def _fused(self, qgroups, k, b, per_event, d_t, te_w, te_b, te_bounds, dt_mode, co_mode) -> dict:
        """One tgx_recent launch over the query groups (no ring plan); with
        co-occurrence the event-major plan puts each event's (src, dst) pair in one
        workgroup, in the layout prepare() launches."""
        g = self.graph
        if co_mode != _lib.TGX_CO_NONE:
            # the extension picks the layout (event_query_groups=-1): every query of
            # an event in its workgroup, or only the (src, dst) pair with the other
            # groups tiled after them (small launches, or more queries per event
            # than a workgroup takes)
            G = sum(per_event)
            return g._query(None, None, k, groups=qgroups, plan_mode=_lib.TGX_PLAN_EVENTS, group=G,
                            num_groups=b, event_query_groups=-1, d_t=d_t, te_w=te_w, te_b=te_b,
                            te_bounds=te_bounds, dt_mode=dt_mode, co_mode=co_mode,
                            want_eids=self.spec.edge_ids)
        return g._query(None, None, k, groups=qgroups, group=self.queries_per_workgroup,
                        d_t=d_t, te_w=te_w, te_b=te_b, te_bounds=te_bounds, dt_mode=dt_mode,
                        want_eids=self.spec.edge_ids)

    @staticmethod
    def _co_occur_from_neighbors(src_nbrs: NeighborData, dst_nbrs: NeighborData) -> Tensor:
        """(B,) float shared-neighbour count from already-gathered neighbours
        (reference pipeline/__init__.py:206-219): the valid src positions (by
        mask) whose id occurs at a valid dst position, computed by
        tgx_co_occurrence with both masks."""
        a = src_nbrs.neighbor_ids.to(torch.int32).contiguous()
        c = dst_nbrs.neighbor_ids.to(torch.int32).contiguous()
        am = src_nbrs.mask.to(torch.bool).contiguous()
        cm = dst_nbrs.mask.to(torch.bool).contiguous()
        P, K = a.shape
        if c.shape != (P, K) or am.shape != (P, K) or cm.shape != (P, K):
            raise ValueError("src and dst neighbours must have the same (B, K) shape")
        dev = a.device
        a_cnt = torch.empty((P, K, 2), dtype=torch.int32, device=dev)
        c_cnt = torch.empty((P, K, 2), dtype=torch.int32, device=dev)
        pair = torch.empty((P,), dtype=torch.float32, device=dev)
        if P and K:
            rc = _lib.lib().tgx_co_occurrence(a.data_ptr(), c.data_ptr(), am.data_ptr(), cm.data_ptr(),
                                              P, K, a_cnt.data_ptr(), c_cnt.data_ptr(),
                                              pair.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
            _lib.check(rc, "tgx_co_occurrence")
        else:
            pair.zero_()
        return pair


from tgengine_amd.pipeline.async_pipeline import AsyncDataPipeline  # noqa: E402

__all__ = ["DataPipeline", "AsyncDataPipeline", "cosine_time_weights", "event_plan"]
