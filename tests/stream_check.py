"""Lock-step parity harness: the HIP streaming loop against the CPU oracle.

Loop per batch i (BASELINE regime): prepare(batch i) -> advance(batch i) on a
graph created empty, so the CSR is frozen empty and all state lives in the
ring.  The oracle replays every advance; queries are compared on the batches
listed in ``check``.  Integer, id, time, mask and feature outputs must be
bit-identical; time encodings within ``te_atol`` of cos of the exact fp32
argument.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import spec as O  # noqa: E402
from tgengine_amd import TemporalGraph  # noqa: E402
from tgengine_amd.synthetic import (CONFIGS, gen_batch, key_multiplier_ok, make_graph,  # noqa: E402,F401
                                    make_pipeline, to_raw)

TE_ATOL = 1e-6


def feats_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def queries_of(bt):
    b = len(bt["src"])
    neg = bt["neg"].reshape(-1)
    n_neg = neg.shape[0] // b
    nodes = np.concatenate([bt["src"], bt["dst"], neg])
    qt = np.concatenate([bt["time"], bt["time"], np.repeat(bt["time"], n_neg)])
    return nodes, qt


class Mismatch(AssertionError):
    pass


def _eq(name, got, exp, where):
    if got.shape != exp.shape:
        raise Mismatch(f"{where}: {name} shape {got.shape} != {exp.shape}")
    if not np.array_equal(got, exp):
        bad = np.argwhere(got != exp)
        raise Mismatch(f"{where}: {name} differs at {len(bad)} positions, first {bad[:3].tolist()}")


def compare_prepared(cfg, pb, bt, ring, w, where, with_te=True, csr=None):
    """Compare one PreparedBatch with the oracle on the same CSR and ring state."""
    b = len(bt["src"])
    K = cfg.k
    d = cfg.feat_dim
    fdt = np.uint16 if cfg.feat_dtype == "bf16" else np.float32
    nodes, qt = queries_of(bt)
    nb = O.recent(nodes, qt, K, csr, ring, d, fdt)
    groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
    ids = np.concatenate([g.neighbor_ids.cpu().numpy() for g in groups])
    tms = np.concatenate([g.timestamps.cpu().numpy() for g in groups])
    msk = np.concatenate([g.mask.cpu().numpy() for g in groups])
    fts = np.concatenate([feats_np(g.edge_feats) for g in groups])
    _eq("ids", ids, nb.ids, where)
    _eq("times", tms.view(np.int64), nb.times.view(np.int64), where)
    _eq("mask", msk, nb.mask, where)
    _eq("feats", fts.view(np.uint32 if fdt == np.float32 else np.uint16),
        nb.feats.view(np.uint32 if fdt == np.float32 else np.uint16), where)
    stats = {"valid": int(nb.mask.sum()), "queries": len(nodes)}
    if with_te:
        te = np.concatenate([g.time_enc.cpu().numpy() for g in groups])
        exact = O.time_encode_exact(O.dt_dygformer(qt, nb.times), w, nb.mask)
        err = float(np.max(np.abs(te.astype(np.float64) - exact))) if te.size else 0.0
        if not err <= TE_ATOL:
            raise Mismatch(f"{where}: time encoding max abs error {err:.3g} > {TE_ATOL}")
        pad = ~nb.mask
        if np.any(te[pad] != 0.0):
            raise Mismatch(f"{where}: padding time encodings are not zero")
        stats["te_max_err"] = err
    if cfg.co_occurrence:
        a, c = nb.ids[:b], nb.ids[b:2 * b]
        a_cnt, c_cnt = O.co_occurrence_freq(a, c)
        ga, gc = pb.co_occurrence_freq
        _eq("co_a", ga.cpu().numpy(), a_cnt, where)
        _eq("co_c", gc.cpu().numpy(), c_cnt, where)
        pair = O.co_pair_count(a, nb.mask[:b], c, nb.mask[b:2 * b])
        _eq("co_pair", pb.co_occurrence.cpu().numpy(), pair, where)
    return stats


def compare_ring(g: TemporalGraph, ring: O.Ring, rows: np.ndarray, where):
    rows = np.unique(rows)
    rt = torch.from_numpy(rows).to(g.device)
    _eq("ring ids", g._ov_ids[rt].cpu().numpy(), ring.ids[rows], where)
    _eq("ring times", g._ov_times[rt].cpu().numpy().view(np.int64), ring.times[rows].view(np.int64), where)
    gf = feats_np(g._ov_feats[rt])
    _eq("ring feats", gf.view(np.uint32 if gf.dtype == np.float32 else np.uint16),
        ring.feats[rows].view(np.uint32 if gf.dtype == np.float32 else np.uint16), where)
    _eq("ring write_pos", g._ov_write_pos.cpu().numpy(), ring.wp, where)


def run(cfg_name: str, n_batches: int, check: set, ring_check_every: int = 0,
        log=print, cfg=None) -> dict:
    """Stream ``n_batches`` batches; compare queries on ``check`` batches."""
    cfg = cfg or CONFIGS[cfg_name]
    fdt = np.uint16 if cfg.feat_dtype == "bf16" else np.float32
    g = make_graph(cfg)
    pipe = make_pipeline(cfg, g)
    ring = O.Ring.empty(cfg.num_nodes, cfg.buffer_size, cfg.feat_dim, fdt)
    w = O.time_weights(100)
    tot = {"valid": 0, "queries": 0, "te_max_err": 0.0, "checked": 0}
    for i in range(n_batches):
        bt = gen_batch(cfg, i)
        assert key_multiplier_ok(bt["time"], len(bt["src"]))
        rb = to_raw(cfg, bt)
        pb = pipe.prepare(rb)
        if i in check:
            st = compare_prepared(cfg, pb, bt, ring if i > 0 else None, w, f"{cfg.name} batch {i}")
            tot["valid"] += st["valid"]
            tot["queries"] += st["queries"]
            tot["te_max_err"] = max(tot["te_max_err"], st.get("te_max_err", 0.0))
            tot["checked"] += 1
        g.advance(rb.src, rb.dst, rb.time, rb.edge_feat)
        O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], bt["feat"])
        if ring_check_every and (i % ring_check_every == ring_check_every - 1 or i == n_batches - 1):
            compare_ring(g, ring, np.concatenate([bt["src"], bt["dst"]]), f"{cfg.name} ring after {i}")
    st = g.status()
    if any(st.values()):
        raise Mismatch(f"{cfg.name}: device diagnostics {st}")
    tot["graph"] = g
    tot["ring"] = ring
    return tot
