"""Benchmark of the fused temporal data pipeline on one MI355X.

A step is one pass of the hot path over one batch of the synthetic stream:
``DataPipeline.prepare(batch i)`` (fused gather + feature rows + 100-d cosine
time encoding [+ co-occurrence]) followed by ``TemporalGraph.advance(batch i)``
(ring update), on a graph created empty -- the BASELINE streaming regime.  The
whole stream window is staged in HBM before timing.

Batches: W warm-up, then the timed region of K steps (``value`` = prepared
queries/s over its wall clock between two device synchronisations, nothing but
the hot path inside), then a roofline window: the fused prepare kernels of the
next R batches on the ring state the timed region left, captured in a HIP graph
and replayed between two HIP events on the launch stream; ``roofline.achieved``
= algorithmic bytes per launch over the mean launch time.  Then the CPU baseline: the torch-CPU restatement of the reference
path run on the same ring state for a bounded window of following batches (its
outputs must equal the GPU's).
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
METRIC = "prepared queries/sec (K-nbr gather+time-enc); achieved HBM GB/s % of peak"


class _no_gc:
    """Python's cyclic garbage collector off inside a host-timed region (as timeit
    does): a collection triggered by the steps' allocations lands at a random step
    and measured as 1-2 us per step of spread over a 20-step window.  No collection
    is forced before (a full one leaves the host's caches cold for the first
    steps: 27 -> 34 us per step over 20); the collector is back on afterwards."""

    def __enter__(self):
        self.was = gc.isenabled()
        gc.disable()

    def __exit__(self, *exc):
        if self.was:
            gc.enable()
        return False


def bytes_per_batch(cfg, Q: int, V: int, pairs: int, d_t: int = 100) -> int:
    """Algorithmic bytes of one prepare launch: per query R = 16 + B*12 + V_q*d*s_f,
    W = K*13 + K*d*s_f + K*d_t*4, plus 16*K per co-occurrence pair."""
    s_f = cfg.feat_bytes
    d, K, B = cfg.feat_dim, cfg.k, cfg.buffer_size
    r = Q * (16 + B * 12) + V * d * s_f
    w = Q * (K * 13 + K * d * s_f + K * d_t * 4)
    return int(r + w + pairs * 16 * K)


def stage_stream(cfg, first: int, count: int, torch, device):
    from tgengine_amd.synthetic import gen_batch
    bts = [gen_batch(cfg, i) for i in range(first, first + count)]
    cat = lambda k: np.concatenate([bt[k] for bt in bts])  # noqa: E731
    dev = {k: torch.from_numpy(cat(k)).to(device) for k in ("src", "dst", "time", "neg")}
    feat = torch.from_numpy(cat("feat"))
    if cfg.feat_dtype == "bf16":
        feat = feat.view(torch.bfloat16)
    dev["feat"] = feat.to(device)
    lens = [len(bt["src"]) for bt in bts]
    return dev, lens, bts


def measure_ceilings(torch, device, launch_bytes: int, log) -> dict:
    """HBM ceilings of plain device kernels, each the best of 5 event-timed
    repetitions after a warm-up: at 1 GiB and at the gather launch's byte count, a
    copy (the runtime's copy kernel, reads + writes the size), an elementwise copy
    (torch's vectorized elementwise kernel, `neg` into another buffer) and a
    store-only fill; then a row gather of the large-row config's shape: 1 KB rows
    at random from a 6.55 GB table (100,000 nodes x 64 slots, the rows read as
    16-byte elements) into a 1 GiB output."""
    out = {}

    def timed(key, fn, moved):
        fn()
        torch.cuda.synchronize()
        best = None
        for _ in range(5):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
        out[key] = {"bytes": moved, "us": best * 1e3, "GB/s": moved / (best * 1e-3) / 1e9}
        log(f"ceiling {key}: {moved / 1e6:.1f} MB in {best * 1e3:.1f} us = "
            f"{moved / (best * 1e-3) / 1e9:.0f} GB/s")

    for name, nbytes in (("1GiB", 1 << 30), ("launch", max(launch_bytes, 1 << 20))):
        n = nbytes // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        timed(f"copy_{name}", lambda: dst.copy_(src), 2 * n * 4)
        timed(f"elementwise_copy_{name}", lambda: torch.neg(src, out=dst), 2 * n * 4)
        timed(f"store_{name}", lambda: dst.fill_(2.0), n * 4)
        del src, dst
        torch.cuda.synchronize()
    rows = 1 << 20
    table = torch.zeros(100_000 * 64, 64, dtype=torch.complex128, device=device)
    idx = torch.randint(0, table.shape[0], (rows,), device=device)
    got = torch.empty(rows, 64, dtype=torch.complex128, device=device)
    timed("row_gather_1KB_1GiB", lambda: torch.index_select(table, 0, idx, out=got),
          2 * rows * 1024 + rows * 8)
    del table, idx, got
    torch.cuda.synchronize()
    return out


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, g, pipe, first, seconds, torch, log, last):
    """Time the torch-CPU restatement of the reference path on batches first.. of the
    stream, starting from the GPU ring state; its outputs must equal the GPU's on
    every batch (ids, timestamps, masks, rows, encodings), and the oracle's
    (oracle/spec.py) on the first batch.

    Two legs: the job's CPU share (OMP_NUM_THREADS where set, else the CPUs in
    this process's affinity mask; torch threads set to that count) for
    ``seconds``, then one thread for a third of that on the following batches.
    os.cpu_count() is reported beside it: on a shared GPU box it counts the whole
    host, not the CPUs this job was given."""
    from oracle import spec
    from oracle.refpath_torch import RefPathCPU
    from tgengine_amd.synthetic import gen_batch, to_raw
    cpu = RefPathCPU(cfg.num_nodes, cfg.feat_dim, cfg.buffer_size)
    cpu.ids.copy_(g._ov_ids.cpu())
    cpu.times.copy_(g._ov_times.cpu())
    cpu.feats.copy_(g._ov_feats.float().cpu())
    cpu.wp.copy_(g._ov_write_pos.cpu())
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    # the job's CPU share: OMP_NUM_THREADS where the box sets it (the GPU boxes
    # give each GPU job 16 CPUs whatever the host counts), else the affinity mask
    omp = os.environ.get("OMP_NUM_THREADS", "")
    share = min(int(omp), affinity) if omp.isdigit() and int(omp) > 0 else affinity
    prev_threads = torch.get_num_threads()
    state = {"i": first}
    want = {}

    def oracle_check(i, bt, src, dst, neg, tt):
        """The oracle's gather + encodings of batch i on the ring state the CPU
        restatement starts from (queries [src, dst, neg row-major])."""
        # views of the CPU ring (read only here; the restatement runs afterwards)
        ring = spec.Ring(ids=cpu.ids.numpy(), times=cpu.times.numpy(), feats=cpu.feats.numpy(),
                         wp=cpu.wp.numpy())
        nodes = np.concatenate([bt["src"], bt["dst"], bt["neg"].reshape(-1)])
        per = bt["neg"].shape[1] if bt["neg"].ndim > 1 else 1
        qt = np.concatenate([bt["time"], bt["time"], np.repeat(bt["time"], per)])
        o = spec.recent(nodes, qt, cfg.k, None, ring, cfg.feat_dim)
        te = spec.time_encode_exact(spec.dt_dygformer(qt, o.times), spec.time_weights(100), o.mask)
        want.update(o=o, te=te)

    def oracle_compare(i, out):
        o = want["o"]
        same = (np.array_equal(out["ids"].numpy(), o.ids) and np.array_equal(out["mask"].numpy(), o.mask)
                and np.array_equal(out["times"].numpy().view(np.int64), o.times.view(np.int64))
                and np.array_equal(out["feats"].numpy(), o.feats))
        err = float(np.abs(out["te"].double().numpy() - want["te"]).max()) if o.ids.size else 0.0
        if not same or err > 1e-6:
            raise RuntimeError(f"CPU baseline and oracle disagree at batch {i} (te error {err:.2e})")
        log(f"cpu baseline: batch {i} equal to the oracle (te max error {err:.2e})")

    def leg(threads, budget):
        torch.set_num_threads(threads)
        spent = 0.0
        queries = batches = 0
        start = state["i"]
        while (spent < budget or batches < 2) and state["i"] < last:
            i = state["i"]
            bt = gen_batch(cfg, i)
            rb = to_raw(cfg, bt)
            pb = pipe.prepare(rb)
            src = torch.from_numpy(bt["src"])
            dst = torch.from_numpy(bt["dst"])
            tt = torch.from_numpy(bt["time"])
            neg = torch.from_numpy(bt["neg"])
            f32 = torch.from_numpy(bt["feat"])
            if cfg.feat_dtype == "bf16":
                f32 = f32.view(torch.bfloat16).float()
            if i == first:
                oracle_check(i, bt, src, dst, neg, tt)
            t0 = time.perf_counter()
            out = cpu.prepare(src, dst, neg, tt, cfg.k, co=cfg.co_occurrence)
            cpu.advance(src, dst, tt, f32)
            spent += time.perf_counter() - t0
            if i == first:
                oracle_compare(i, out)
            # parity of the CPU restatement with the GPU on this full-size window
            groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
            gids = torch.cat([x.neighbor_ids.cpu() for x in groups])
            gtimes = torch.cat([x.timestamps.cpu() for x in groups])
            gmask = torch.cat([x.mask.cpu() for x in groups])
            gfeat = torch.cat([x.edge_feats.float().cpu() for x in groups])
            gte = torch.cat([x.time_enc.cpu() for x in groups])
            if not (torch.equal(gids, out["ids"]) and torch.equal(gmask, out["mask"])
                    and torch.equal(gtimes.view(torch.int64), out["times"].view(torch.int64))
                    and torch.equal(gfeat, out["feats"])):
                raise RuntimeError(f"CPU baseline and GPU disagree at batch {i}")
            te_err = float((gte.double() - out["te"].double()).abs().max()) if gte.numel() else 0.0
            if te_err > 2e-6:
                raise RuntimeError(f"time encodings differ by {te_err} at batch {i}")
            g.advance(rb.src, rb.dst, rb.time, rb.edge_feat)
            queries += len(bt["src"]) * cfg.queries_per_event
            batches += 1
            state["i"] += 1
        log(f"cpu baseline: {batches} batches, {queries} queries in {spent:.2f}s on {threads} threads")
        return queries, spent, start, batches

    q_n, s_n, b0, nb = leg(share, seconds)
    q_1, s_1, b1, nb1 = leg(1, seconds / 3)
    torch.set_num_threads(prev_threads)
    return {"value": q_n / s_n, "unit": "prepared queries/s", "cores": share,
            "kind": "port",
            "sample": (f"{cfg.name} batches {b0}..{b0 + nb - 1} ({q_n} queries, prepare+advance) "
                       f"from the GPU ring state after batch {b0 - 1}; outputs equal to the GPU's "
                       f"(ids, timestamps, masks, rows, encodings), and to the oracle's on batch {b0}"),
            "batches": nb, "threads": share, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": affinity, "cpu_model": cpu_model(),
            "value_1thread": q_1 / s_1 if s_1 > 0 else None,
            "sample_1thread": f"{cfg.name} batches {b1}..{b1 + nb1 - 1} ({q_1} queries) on 1 thread"}


def run_rows(a, log) -> None:
    """--rows: the functions beside the streaming path, on the C3 graph (1M nodes,
    16-d bf16 rows): freeze_csr (tgx_csr_build) of a pre-freeze prefix of the
    stream (as generated, with its times floored, and with its times permuted
    within each batch: the three builds), recent() on the frozen CSR, recent_2hop() and HistoricalNegPool
    update + sample.  Each is timed on the device (HIP events; the gathers and the
    pool as graph replays of successive batches) and priced against its
    algorithmic bytes, and the oracle's restatement of the same function is timed
    on a bounded sample whose outputs are compared with the device's.  One JSON
    line per row."""
    import numpy as np
    import torch
    from oracle import spec  # the CPU legs only
    from tgengine_amd.pipeline.negatives import HistoricalNegPool
    from tgengine_amd.synthetic import CONFIGS, make_graph
    cfg = CONFIGS["c3"]
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    P, R, S = a.rows_batches, 200, a.rows_cpu_batches
    N, d, K = cfg.num_nodes, cfg.feat_dim, cfg.k
    rb = d * cfg.feat_bytes
    t0 = time.time()
    dev, lens, bts = stage_stream(cfg, 0, P + R, torch, device)
    offs = np.concatenate([[0], np.cumsum(lens)])
    log(f"rows: staged {P + R} batches in {time.time() - t0:.1f}s")

    def ev(i):
        s_, e_ = int(offs[i]), int(offs[i + 1])
        return dev["src"][s_:e_], dev["dst"][s_:e_], dev["time"][s_:e_], dev["feat"][s_:e_]

    def filled(n):
        g = make_graph(cfg)
        for i in range(n):
            g.advance(*ev(i))
        torch.cuda.synchronize()
        return g

    def timed_ms(fn):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    def replay_ms(calls):
        """HIP-event time of one replay of a graph that captures calls()."""
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            kept = calls()
        graph.replay()
        ms = min(timed_ms(graph.replay) for _ in range(3))
        return ms, kept

    def line(row, workload, unit, value, ms, nbytes, cpu, parity, extra=None):
        gbs = nbytes / (ms * 1e-3) / 1e9
        out = {"row": row, "metric": f"{unit} ({row})", "value": value, "unit": unit,
               "ms_per_call": ms, "workload": workload,
               "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": gbs / PEAK_HBM_GBS, "bytes_per_call": nbytes},
               "cpu_baseline": cpu, "parity": parity}
        out.update(extra or {})
        print(json.dumps(out), flush=True)

    def gather_bytes(masks, k):
        """recent() without encodings: per query the CSR offsets (16 B) and V taken
        entries (id, time, row) read; K slots (id, time, row, mask) written."""
        q = sum(int(m.shape[0]) for m in masks)
        v = sum(int(m.sum()) for m in masks)
        return q * 16 + v * (12 + rb) + q * k * (13 + rb), q, v

    # ---- freeze_csr: P batches frozen on a fresh graph, three times ----
    E = int(offs[P])
    gw = filled(4)
    gw.freeze_csr()
    del gw
    fr = []
    for rep in range(3):
        g = filled(P)
        fr.append(timed_ms(g.freeze_csr))
        if rep < 2:
            del g
            torch.cuda.synchronize()
    ms = min(fr)
    fbytes = E * (24 + rb) + 2 * E * (12 + rb) + (N + 1) * 8
    # CPU: the oracle's freeze of the first S batches, compared with a device freeze of them
    evs = [(bt["src"], bt["dst"], bt["time"], bt["feat"], int(offs[i])) for i, bt in enumerate(bts[:S])]
    c0 = time.perf_counter()
    csr_s = spec.csr_freeze(N, d, evs, feat_dtype=np.uint16)
    cs = time.perf_counter() - c0
    gs = filled(S)
    gs.freeze_csr()
    same = (np.array_equal(gs._offsets.cpu().numpy(), csr_s.offsets)
            and np.array_equal(gs._nbr_ids.cpu().numpy(), csr_s.ids)
            and np.array_equal(gs._nbr_times.cpu().numpy().view(np.int64), csr_s.times.view(np.int64))
            and np.array_equal(gs._nbr_feats.view(torch.int16).cpu().numpy().view(np.uint16), csr_s.feats))
    del gs
    if not same:
        raise RuntimeError("rows: the device CSR of the sample differs from the oracle's")
    ES = int(offs[S])
    line("csr_build", f"freeze_csr of C3 batches 0..{P - 1}: {E} events, {2 * E} directed entries, "
         f"{N} nodes, {d}-d bf16 rows", "events/s", E / (ms * 1e-3), ms, fbytes,
         {"value": ES / cs, "unit": "events/s", "cores": 1, "kind": "port",
          "sample": f"oracle.spec.csr_freeze (numpy) of batches 0..{S - 1} ({ES} events)"},
         f"CSR arrays of batches 0..{S - 1} equal to the oracle's", {"reps_ms": fr})
    log(f"rows: csr_build {ms:.2f} ms for {E} events")

    # ---- the same freeze with tied times (floored to whole numbers: runs of equal
    # times, no time passes) and with times permuted within each batch (the build
    # order sorted by time first) ----
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    perm = torch.cat([torch.randperm(int(e_ - s_), device=device, generator=gen) + int(s_)
                      for s_, e_ in zip(offs[:P], offs[1:P + 1])])
    for row, how, tv in (("csr_build_tied", "times floored to whole numbers", torch.floor(dev["time"][:E])),
                         ("csr_build_shuffled", "times permuted within each batch", dev["time"][perm])):
        def filled_v(n, tv=tv):
            gv = make_graph(cfg)
            for i in range(n):
                s_, e_ = int(offs[i]), int(offs[i + 1])
                gv.advance(dev["src"][s_:e_], dev["dst"][s_:e_], tv[s_:e_], dev["feat"][s_:e_])
            torch.cuda.synchronize()
            return gv
        frv = []
        for rep in range(3):
            gv = filled_v(P)
            frv.append(timed_ms(gv.freeze_csr))
            mode = gv._csr_build_mode
            del gv
            torch.cuda.synchronize()
        msv = min(frv)
        tv_host = tv[:ES].cpu().numpy()
        evs = [(bt["src"], bt["dst"], tv_host[int(offs[i]):int(offs[i + 1])], bt["feat"], int(offs[i]))
               for i, bt in enumerate(bts[:S])]
        c0 = time.perf_counter()
        csr_v = spec.csr_freeze(N, d, evs, feat_dtype=np.uint16)
        cv = time.perf_counter() - c0
        gs = filled_v(S)
        gs.freeze_csr()
        same = (np.array_equal(gs._offsets.cpu().numpy(), csr_v.offsets)
                and np.array_equal(gs._nbr_ids.cpu().numpy(), csr_v.ids)
                and np.array_equal(gs._nbr_times.cpu().numpy().view(np.int64), csr_v.times.view(np.int64))
                and np.array_equal(gs._nbr_feats.view(torch.int16).cpu().numpy().view(np.uint16), csr_v.feats))
        del gs
        if not same:
            raise RuntimeError(f"rows: the device CSR of the {row} sample differs from the oracle's")
        line(row, f"freeze_csr of C3 batches 0..{P - 1} with {how} ({mode} build): {E} events, "
             f"{2 * E} directed entries, {N} nodes, {d}-d bf16 rows", "events/s", E / (msv * 1e-3), msv, fbytes,
             {"value": ES / cv, "unit": "events/s", "cores": 1, "kind": "port",
              "sample": f"oracle.spec.csr_freeze (numpy) of batches 0..{S - 1} ({ES} events)"},
             f"CSR arrays of batches 0..{S - 1} equal to the oracle's", {"reps_ms": frv, "build": mode})
        log(f"rows: {row} {msv:.2f} ms ({mode} build)")

    # ---- recent() on the frozen CSR: the next R batches' src/dst/neg queries ----
    qs = []
    for i in range(P, P + R):
        s_, d_, t_, _ = ev(i)
        neg = dev["neg"][int(offs[i]):int(offs[i + 1])].reshape(-1)
        qs.append((torch.cat([s_, d_, neg]), torch.cat([t_, t_, t_])))
    ref = g.recent(qs[0][0], qs[0][1], K)
    torch.cuda.synchronize()

    def recent_calls():
        return [g.recent(n_, t_, K).mask for (n_, t_) in qs]
    ms, masks = replay_ms(recent_calls)
    ms /= R
    nbytes, q, v = gather_bytes(masks, K)
    nbytes //= R
    # CPU: the oracle's recent() over the full CSR, for the first batch's queries
    evs_all = [(bt["src"], bt["dst"], bt["time"], bt["feat"], int(offs[i])) for i, bt in enumerate(bts[:P])]
    csr_all = spec.csr_freeze(N, d, evs_all, feat_dtype=np.uint16)
    del evs_all
    n0, t0_ = qs[0][0].cpu().numpy(), qs[0][1].cpu().numpy()
    c0 = time.perf_counter()
    o = spec.recent(n0, t0_, K, csr_all, None, d, feat_dtype=np.uint16)
    cs = time.perf_counter() - c0
    same = (np.array_equal(ref.neighbor_ids.cpu().numpy(), o.ids) and np.array_equal(ref.mask.cpu().numpy(), o.mask)
            and np.array_equal(ref.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
            and np.array_equal(ref.edge_feats.view(torch.int16).cpu().numpy().view(np.uint16), o.feats))
    if not same:
        raise RuntimeError("rows: recent() on the frozen CSR differs from the oracle's")
    line("recent_csr", f"recent() of C3 batches {P}..{P + R - 1}'s src/dst/neg ({q // R} queries per call, "
         f"K={K}) on the frozen CSR of batches 0..{P - 1}, mean V {v / q:.2f}", "queries/s", q / (ms * 1e-3 * R),
         ms, nbytes, {"value": len(n0) / cs, "unit": "queries/s", "cores": 1, "kind": "port",
                      "sample": f"oracle.spec.recent (numpy) of batch {P}'s {len(n0)} queries"},
         f"batch {P}'s ids, times, rows and masks equal to the oracle's",
         {"timing": f"HIP event pair around a graph replay of {R} calls"})
    log(f"rows: recent_csr {ms * 1e3:.2f} us per call")

    # ---- recent_2hop(): each next batch's src, k1 = k2 = K ----
    R2 = 50
    ref2 = g.recent_2hop(qs[0][0][:lens[P]], qs[0][1][:lens[P]], K, K)
    torch.cuda.synchronize()

    def hop_calls():
        out = []
        for i in range(R2):
            b_ = lens[P + i]
            r_ = g.recent_2hop(qs[i][0][:b_], qs[i][1][:b_], K, K)
            out += [r_.mask, r_.hop2_mask.reshape(-1, K)]
        return out
    ms, masks = replay_ms(hop_calls)
    ms /= R2
    nbytes, q, v = gather_bytes(masks, K)
    nbytes //= R2
    ns = 500
    n1, t1 = n0[:ns], t0_[:ns]
    c0 = time.perf_counter()
    h1 = spec.recent(n1, t1, K, csr_all, None, d, feat_dtype=np.uint16)
    n2 = np.where(h1.mask, h1.ids, -1).reshape(-1).astype(np.int64)
    h2 = spec.recent(n2, h1.times.reshape(-1), K, csr_all, None, d, feat_dtype=np.uint16)
    cs = time.perf_counter() - c0
    m2 = h2.mask.reshape(ns, K, K)
    same = (np.array_equal(ref2.neighbor_ids[:ns].cpu().numpy(), h1.ids)
            and np.array_equal(ref2.hop2_mask[:ns].cpu().numpy(), m2)
            and np.array_equal(ref2.hop2_ids[:ns].cpu().numpy(), np.where(m2, h2.ids.reshape(ns, K, K), -1)))
    if not same:
        raise RuntimeError("rows: recent_2hop differs from the oracle's composition")
    line("recent_2hop", f"recent_2hop() of C3 batches {P}..{P + R2 - 1}'s src ({lens[P]} queries per call, "
         f"k1=k2={K}: {lens[P] * K} hop-2 queries) on the frozen CSR", "hop-2 queries/s",
         sum(lens[P:P + R2]) * K / (ms * 1e-3 * R2), ms, nbytes,
         {"value": ns * K / cs, "unit": "hop-2 queries/s", "cores": 1, "kind": "port",
          "sample": f"oracle.spec.recent twice (numpy), batch {P}'s first {ns} src queries"},
         f"hop-1 ids and hop-2 ids and masks of batch {P}'s first {ns} queries equal to the oracle's",
         {"timing": f"HIP event pair around a graph replay of {R2} calls (two launches each)"})
    log(f"rows: recent_2hop {ms * 1e3:.2f} us per call")
    del g, csr_all
    torch.cuda.synchronize()

    # ---- HistoricalNegPool: update with batch i's edges, then sample batch i's src ----
    Pp = 512
    pool = HistoricalNegPool(N, Pp, device=str(device), seed=12345)
    for i in range(4):
        s_, d_, _, _ = ev(i)
        pool.update(s_, d_)
        pool.sample(s_)
    torch.cuda.synchronize()

    def pool_calls():
        out = []
        for i in range(4, 4 + R):
            s_, d_, _, _ = ev(i)
            pool.update(s_, d_)
            out.append(pool.sample(s_))
        return out
    ms, _ = replay_ms(pool_calls)
    ms /= R
    nev = sum(lens[4:4 + R]) / R
    nbytes = int(nev * (16 + 8 + 4 + 8) + nev * (8 + 8 + 4 + 8))
    del pool
    torch.cuda.synchronize()
    # CPU: the oracle's edge-by-edge update and sample over the first S2 batches of a
    # fresh pool, compared call by call with a fresh device pool of the same seed
    S2 = min(S, 20)
    pool = HistoricalNegPool(N, Pp, device=str(device), seed=777)
    cp = np.full((N, Pp), -1, np.int32)
    cc = np.zeros(N, np.int64)
    cs = 0.0
    for i in range(S2):
        s_, d_, _, _ = ev(i)
        pool.update(s_, d_)
        got = pool.sample(s_).cpu().numpy()
        c0 = time.perf_counter()
        spec.negpool_update(cp, cc, bts[i]["src"], bts[i]["dst"], 777, 2 * i)
        want = spec.negpool_sample(cp, cc, bts[i]["src"], 777, 2 * i + 1)
        cs += time.perf_counter() - c0
        if not np.array_equal(got, want):
            raise RuntimeError(f"rows: negative pool sample {i} differs from the oracle's")
    if not (np.array_equal(pool._pool.cpu().numpy(), cp) and np.array_equal(pool._count.cpu().numpy(), cc)):
        raise RuntimeError("rows: negative pool state differs from the oracle's")
    del pool, cp
    ES2 = int(offs[S2])
    line("negpool", f"HistoricalNegPool({N} nodes, pool {Pp}): update with a C3 batch's edges, then sample its "
         f"src ({nev:.0f} edges per call, batches 4..{3 + R})", "edges/s", nev / (ms * 1e-3), ms, nbytes,
         {"value": ES2 / cs, "unit": "edges/s", "cores": 1, "kind": "port",
          "sample": f"oracle.spec.negpool_update + negpool_sample (numpy), batches 0..{S2 - 1} ({ES2} edges)"},
         f"every sample of batches 0..{S2 - 1} and the final pool and counts equal to the oracle's",
         {"timing": f"HIP event pair around a graph replay of {R} update + sample pairs"})
    log(f"rows: negpool {ms * 1e3:.2f} us per update + sample")


RING_SHAPES = ("c3", "singletons", "one_node", "groups8", "pairs", "groups10", "groups40", "groups100")


def ring_shape_batch(cfg, name: str, j: int):
    """src, dst of batch j of a 4,000-event ring-update shape on cfg's node range:
    the C3 stream itself, or entries built to give every node the same count (each
    node once, all entries on one node, groups of 8, 2, 10, 40 or 100 entries); the
    node set moves between batches."""
    from tgengine_amd.synthetic import gen_batch
    b = 4000
    i = np.arange(b, dtype=np.int64)
    base = (j * 7919) % (cfg.num_nodes - 10000)
    if name == "c3":
        bt = gen_batch(cfg, 3000 + j, with_feats=False)
        return bt["src"][:b].astype(np.int64), bt["dst"][:b].astype(np.int64)
    groups = {"groups8": 1000, "pairs": b, "groups10": 800, "groups40": 200, "groups100": 80}
    if name == "singletons":
        return base + 2 * i, base + 2 * i + 1
    if name == "one_node":
        return np.full(b, base, np.int64), np.full(b, base, np.int64)
    g = groups[name]
    return base + i % g, base + (i + 7) % g


def run_ring_shapes(a, log) -> None:
    """--ring-shapes: the ring update alone (tgx_ring_append: the plan launch, then
    the commit launch) on the C3 ring (1M nodes, 32 slots, 16-d bf16 rows) for
    4,000-event batches of several shapes, one JSON line each.  Per shape: the
    first 3 batches on an empty ring are compared with the oracle's ring_advance
    (every touched node's slots, times, rows and write position), then 100 appends
    are captured in a HIP graph and replayed between two HIP events, then 100
    batches run through DataPipeline.prepare -> advance (the plan in the gather
    launch, the commit alone; untimed here, so that a kernel trace of this command
    shows the commit of both paths)."""
    import torch
    from oracle import spec  # the CPU legs only
    from tgengine_amd import RawBatch
    from tgengine_amd.synthetic import CONFIGS, make_graph, make_pipeline
    cfg = CONFIGS["c3"]
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    N, d, b, NB = cfg.num_nodes, cfg.feat_dim, 4000, 100
    rng = np.random.default_rng(11)
    shapes = [s for s in a.ring_shapes.split(",") if s]
    for name in shapes:
        if name not in RING_SHAPES:
            raise SystemExit(f"--ring-shapes: unknown shape {name!r} (one of {', '.join(RING_SHAPES)})")
    t_next = 1.0e7
    for name in shapes:
        host, devb = [], []
        for j in range(3 + 2 * NB):
            s_, d_ = ring_shape_batch(cfg, name, j)
            tt = t_next + np.arange(b) * 1e-3
            t_next = float(tt[-1]) + 1.0
            f = (rng.standard_normal((b, d)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
            host.append((s_, d_, tt, f))
            devb.append((torch.from_numpy(s_).to(device), torch.from_numpy(d_).to(device),
                         torch.from_numpy(tt).to(device), torch.from_numpy(f).view(torch.bfloat16).to(device),
                         torch.from_numpy(rng.integers(0, N, b)).to(device)))
        g = make_graph(cfg)
        g.freeze_csr()
        # parity: the first 3 batches on an empty ring against the oracle
        ring = spec.Ring.empty(N, cfg.buffer_size, d, np.uint16)
        ring.times.fill(0.0)  # touch every page before the oracle is timed
        ring.feats.fill(0)
        c0 = time.perf_counter()
        for j in range(3):
            spec.ring_advance(ring, *host[j])
        cpu_s = time.perf_counter() - c0
        for j in range(3):
            g.advance(*devb[j][:4])
        torch.cuda.synchronize()
        touched = np.unique(np.concatenate([np.concatenate(h[:2]) for h in host[:3]]))
        tt_ = torch.from_numpy(touched).to(device)
        same = (np.array_equal(g._ov_ids[tt_].cpu().numpy(), ring.ids[touched])
                and np.array_equal(g._ov_times[tt_].cpu().numpy(), ring.times[touched])
                and np.array_equal(g._ov_feats[tt_].view(torch.int16).cpu().numpy().view(np.uint16),
                                   ring.feats[touched])
                and np.array_equal(g._ov_write_pos[tt_].cpu().numpy(), ring.wp[touched]))
        if not same:
            raise RuntimeError(f"ring-shapes {name}: the ring after 3 batches differs from the oracle's")
        del ring
        # timed: NB appends, captured once and replayed
        for j in range(3, 13):
            g.advance(*devb[j][:4])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for j in range(3, 3 + NB):
                g.advance(*devb[j][:4])
        graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / NB
        del graph
        # the same batches' shape through prepare -> advance (commit alone)
        pipe = make_pipeline(cfg, g)
        for j in range(3 + NB, 3 + 2 * NB):
            s_, d_, t_, f_, n_ = devb[j]
            pipe.prepare(RawBatch(src=s_, dst=d_, time=t_, edge_feat=f_, neg=n_))
            g.advance(s_, d_, t_, f_)
        torch.cuda.synchronize()
        st = g.status()
        if any(st.values()):
            raise RuntimeError(f"ring-shapes {name}: device diagnostics {st}")
        # algorithmic bytes: every event read (ids, time, row), every kept entry
        # written (id, time, row) and every touched node's write position
        kept = distinct = 0
        for s_, d_, _, _ in host[3:3 + NB]:
            u, c = np.unique(np.concatenate([s_, d_]), return_counts=True)
            kept += int(np.minimum(c, cfg.buffer_size).sum())
            distinct += len(u)
        rb = d * cfg.feat_bytes
        nbytes = (NB * b * (24 + rb) + kept * (12 + rb) + distinct * 8) / NB
        gbs = nbytes / (us * 1e-6) / 1e9
        u0, c0_ = np.unique(np.concatenate(host[3][:2]), return_counts=True)
        print(json.dumps({
            "row": "ring_update", "shape": name, "metric": "events/s (ring update alone)",
            "value": b / (us * 1e-6), "unit": "events/s", "us_per_append": us,
            "workload": f"tgx_ring_append of 4,000-event batches on the C3 ring ({N} nodes, "
                        f"{cfg.buffer_size} slots, {d}-d bf16 rows): {len(u0)} nodes per batch, up to "
                        f"{int(c0_.max())} entries per node",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "bytes_per_call": nbytes},
            "cpu_baseline": {"value": 3 * b / cpu_s, "unit": "events/s", "cores": 1, "kind": "port",
                             "sample": "oracle.spec.ring_advance (numpy) of the shape's first 3 batches"},
            "parity": "after 3 batches on an empty ring, every touched node's ids, times, rows and "
                      "write position equal to the oracle's",
            "timing": f"HIP event pair around a graph replay of {NB} appends"}), flush=True)
        log(f"ring-shapes {name}: {us:.2f} us per append")
        del g, pipe, devb
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def run_csr_prepare(a, log) -> None:
    """--csr-prepare: DataPipeline.prepare on a frozen CSR, as the reference's Engine
    runs it (engine/__init__.py:174-195: advance the training events, freeze,
    then prepare batches without advancing), at the shapes of its published
    pipeline timings (docs/performance_report.md:29-31): Wikipedia (K=32),
    Reddit (K=64) and LastFM (K=512, 2-d rows) node and event counts, batch 200,
    one negative per event (600 queries), plus the 100-d cosine time encoding.
    The first 70% of each synthetic stream is frozen; batches of the rest are
    prepared.  Per shape: host-inclusive microseconds per prepare step (outputs
    held to the next step, as a training loop does), the gather kernel's time
    per launch (a HIP graph of R launches replayed between two HIP events), its
    algorithmic bytes against the HBM roofline, and the oracle's restatement on
    one batch (outputs compared, and its time as the CPU baseline).  One JSON
    line per shape."""
    import torch
    from oracle import spec
    from tgengine_amd import RawBatch
    from tgengine_amd.synthetic import ENGINE_SHAPES, make_graph, make_pipeline, num_batches
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    published_ms = {"wikipedia": 1.83, "reddit": 3.69, "lastfm": 1.70}
    for name in a.csr_shapes.split(","):
        cfg = ENGINE_SHAPES[name]
        nb = num_batches(cfg)
        ntrain = int(0.7 * nb)
        W, S, R = 20, min(a.csr_steps, nb - ntrain - 20), min(200, nb - ntrain)
        t0 = time.time()
        dev, lens, bts = stage_stream(cfg, 0, nb, torch, device)
        offs = np.concatenate([[0], np.cumsum(lens)])

        def raw(i):
            s_, e_ = int(offs[i]), int(offs[i + 1])
            return RawBatch(src=dev["src"][s_:e_], dst=dev["dst"][s_:e_], time=dev["time"][s_:e_],
                            edge_feat=dev["feat"][s_:e_], neg=dev["neg"][s_:e_])
        g = make_graph(cfg)
        for i in range(ntrain):
            r_ = raw(i)
            g.advance(r_.src, r_.dst, r_.time, r_.edge_feat)
        torch.cuda.synchronize()
        f0 = time.perf_counter()
        g.freeze_csr()
        torch.cuda.synchronize()
        freeze_ms = (time.perf_counter() - f0) * 1e3
        pipe = make_pipeline(cfg, g)
        pipe.plan_updates = False  # nothing is advanced after the freeze
        raws = [raw(i) for i in range(ntrain, nb)]
        log(f"{name}: staged {nb} batches, froze {ntrain} ({int(offs[ntrain])} events) in "
            f"{freeze_ms:.1f} ms, {time.time() - t0:.1f}s so far")
        # host-inclusive steps
        pb = None
        for i in range(W):
            pb = pipe.prepare(raws[i])
        torch.cuda.synchronize()
        with _no_gc():
            h0 = time.perf_counter()
            for i in range(W, W + S):
                pb = pipe.prepare(raws[i])
            torch.cuda.synchronize()
            step_us = (time.perf_counter() - h0) / S * 1e6
        del pb
        # kernel time per launch: the first R prepare launches, graph-replayed
        args = pipe.launch_args(raws[0])
        masks = []
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(R):
                masks.append(tuple(pipe.launch(raws[i], args)["mask"]))
        graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        kern_us = e0.elapsed_time(e1) * 1e3 / R
        del graph
        Q = sum(int(m.shape[0]) for ms in masks for m in ms)
        V = sum(int(m.sum()) for ms in masks for m in ms)
        rb_ = cfg.feat_dim * cfg.feat_bytes
        # per query: query id + time and its CSR offsets read, V entries (id, time,
        # row) read; K slots of id, time, mask, row and d_t encodings written
        nbytes = (Q * (16 + 16) + V * (12 + rb_) + Q * cfg.k * (13 + rb_ + 4 * cfg.d_t)) / R
        gbs = nbytes / (kern_us * 1e-6) / 1e9
        # parity and CPU baseline: the oracle on the first prepared batch
        evs = [(bt["src"], bt["dst"], bt["time"], bt["feat"], int(offs[i])) for i, bt in enumerate(bts[:ntrain])]
        csr = spec.csr_freeze(cfg.num_nodes, cfg.feat_dim, evs, np.float32)
        bt = bts[ntrain]
        nodes = np.concatenate([bt["src"], bt["dst"], bt["neg"]])
        qt = np.concatenate([bt["time"]] * 3)
        c0 = time.perf_counter()
        o = spec.recent(nodes, qt, cfg.k, csr, None, cfg.feat_dim)
        te = spec.time_encode_exact(spec.dt_dygformer(qt, o.times), spec.time_weights(cfg.d_t), o.mask)
        cpu_s = time.perf_counter() - c0
        pb = pipe.prepare(raws[0])
        groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
        got = {k: torch.cat([getattr(x, f) for x in groups]).cpu().numpy()
               for k, f in (("ids", "neighbor_ids"), ("times", "timestamps"), ("mask", "mask"),
                            ("feats", "edge_feats"), ("te", "time_enc"))}
        same = (np.array_equal(got["ids"], o.ids) and np.array_equal(got["mask"], o.mask)
                and np.array_equal(got["times"].view(np.int64), o.times.view(np.int64))
                and np.array_equal(got["feats"], o.feats))
        te_err = float(np.abs(got["te"] - te).max())
        if not same or te_err > 1e-6:
            raise RuntimeError(f"csr prepare {name}: device and oracle differ (te error {te_err:.2e})")
        del csr, evs, pb, got
        line = {"row": f"prepare_csr_{name}",
                "metric": "prepared queries/s (DataPipeline.prepare on a frozen CSR, Engine shape)",
                "value": 600 / (step_us * 1e-6), "unit": "prepared queries/s",
                "us_per_step": step_us, "kernel_us_per_launch": kern_us,
                "workload": (f"{name}-shaped synthetic stream: {cfg.num_nodes} nodes, {cfg.num_events} events, "
                             f"{ntrain} batches of 200 frozen, then prepare() of the next batches without "
                             f"advancing: 600 queries (src, dst, 1 negative), K={cfg.k}, {cfg.feat_dim}-d f32 "
                             f"rows, 100-d time encoding; mean V {V / Q:.1f}"),
                "freeze_ms": freeze_ms,
                "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": gbs / PEAK_HBM_GBS, "bytes_per_launch": nbytes,
                             "timing": f"HIP event pair around a graph replay of {R} launches"},
                "cpu_baseline": {"value": len(nodes) / cpu_s, "unit": "prepared queries/s", "cores": 1,
                                 "kind": "port",
                                 "sample": f"oracle.spec.recent + time_encode_exact (numpy) of batch {ntrain}"},
                "parity": f"batch {ntrain}'s ids, times, masks and rows equal to the oracle's, encodings "
                          f"within {te_err:.1e}",
                "reference_published_ms_per_step": published_ms[name],
                "reference_published_note": "Pipeline/Sampling per step on an RTX 4080, DyGFormer spec "
                                            "(no time encoding), docs/performance_report.md:47-74"}
        print(json.dumps(line), flush=True)
        log(f"{name}: {step_us:.1f} us/step, kernel {kern_us:.2f} us, {gbs:.0f} GB/s")
        del g, pipe, raws, dev, bts
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=600)
    ap.add_argument("--warmup", type=int, default=1400)
    ap.add_argument("--config", default="c3")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--queries-per-workgroup", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--roofline-steps", type=int, default=200,
                    help="batches after the timed region whose prepare kernels are timed back to back")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after timing, run a plain device copy of this size (PMC byte calibration)")
    ap.add_argument("--rows", action="store_true",
                    help="instead of the streaming step, time the rows beside it (freeze_csr, recent() "
                         "on the frozen CSR, recent_2hop, the negative pool), one JSON line each")
    ap.add_argument("--rows-batches", type=int, default=2500,
                    help="--rows: C3 batches frozen into the CSR")
    ap.add_argument("--rows-cpu-batches", type=int, default=100,
                    help="--rows: C3 batches in the oracle's samples")
    ap.add_argument("--csr-prepare", action="store_true",
                    help="instead of the streaming step, time DataPipeline.prepare on a frozen CSR at the "
                         "reference's published Engine shapes (Wikipedia, Reddit, LastFM), one JSON line each")
    ap.add_argument("--csr-shapes", default="wikipedia,reddit,lastfm")
    ap.add_argument("--csr-steps", type=int, default=500)
    ap.add_argument("--ring-shapes", default="", nargs="?", const=",".join(RING_SHAPES),
                    help="instead of the streaming step, time the ring update alone for 4,000-event "
                         "batches of these shapes (all when given without a list), one JSON line each")
    ap.add_argument("--ceilings", action="store_true",
                    help="after timing, measure the device's copy, store and row-gather ceilings "
                         "(plain torch kernels at 1 GiB and at the gather's byte count) and report them")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only: the fused pipeline path has no multi-GPU mode "
              f"(asked for --gpus {a.gpus}); see DESIGN.md for how it would shard.", file=sys.stderr)
        sys.exit(2)
    log = (lambda *x: None) if a.quiet else (lambda *x: print(*x, file=sys.stderr, flush=True))
    if a.rows:
        run_rows(a, log)
        return
    if a.csr_prepare:
        run_csr_prepare(a, log)
        return
    if a.ring_shapes:
        run_ring_shapes(a, log)
        return

    import torch
    from tgengine_amd.synthetic import CONFIGS, make_graph, make_pipeline, num_batches
    cfg = CONFIGS[a.config]
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    # batches: W warm-up, K timed (value), R roofline window (kernel-dispatch events)
    avail = num_batches(cfg)
    # a short stream (C1) keeps a few batches after the timed work for the CPU baseline,
    # also under --no-cpu, so that a profiling run times the same window as the default run
    reserve = min(64, avail // 10)
    # a short stream still gets a short warm-up (the first batches freeze the CSR,
    # build the launch context and grow the allocator's pools)
    w0 = min(a.warmup, 32, avail // 8)
    K = min(a.steps, max(1, avail - reserve - w0))
    R = min(a.roofline_steps, max(0, avail - K - reserve - w0))
    W = min(a.warmup, max(0, avail - K - R - reserve))
    total = W + K + R
    t0 = time.time()
    dev, lens, bts = stage_stream(cfg, 0, total, torch, device)
    log(f"{cfg.name}: staged {total} batches ({sum(lens)} events) in {time.time() - t0:.1f}s")
    for bt in bts:
        from tgengine_amd.synthetic import key_multiplier_ok
        assert key_multiplier_ok(bt["time"], len(bt["src"]))
    del bts

    g = make_graph(cfg)
    pipe = make_pipeline(cfg, g)
    pipe.queries_per_workgroup = a.queries_per_workgroup
    from tgengine_amd import RawBatch
    offs = np.concatenate([[0], np.cumsum(lens)])
    n_neg = cfg.n_neg

    def raw(i):
        s, e = int(offs[i]), int(offs[i + 1])
        neg = dev["neg"][s:e] if n_neg == 1 else dev["neg"][s:e]
        return RawBatch(src=dev["src"][s:e], dst=dev["dst"][s:e], time=dev["time"][s:e],
                        edge_feat=dev["feat"][s:e], neg=neg)

    raws = [raw(i) for i in range(total)]
    # warm-up steps exactly as the timed ones: each step's outputs live until the
    # next step's replace them, so the caching allocator holds both output blocks
    # before timing starts
    pb = None
    for i in range(W):
        pb = pipe.prepare(raws[i])
        g.advance(raws[i].src, raws[i].dst, raws[i].time, raws[i].edge_feat)
    del pb
    torch.cuda.synchronize()
    log(f"warm-up {W} batches done")

    # timed region: K steps, nothing but the hot path between the synchronisations;
    # every step's outputs are dropped before the next, as in a training loop, so
    # the caching allocator hands the same blocks back each step
    host_prep = host_adv = 0.0
    total_q = 0
    torch.cuda.synchronize()
    with _no_gc():
        t_start = time.perf_counter()
        for i in range(W, W + K):
            h0 = time.perf_counter()
            pb = pipe.prepare(raws[i])
            h1 = time.perf_counter()
            g.advance(raws[i].src, raws[i].dst, raws[i].time, raws[i].edge_feat)
            host_adv += time.perf_counter() - h1
            host_prep += h1 - h0
            total_q += lens[i] * cfg.queries_per_event
        del pb
        torch.cuda.synchronize()
        wall = time.perf_counter() - t_start

    # roofline window: the prepare kernels of the next R batches of the stream on the
    # ring state the timed region left, captured once in a HIP graph and replayed
    # between two HIP events on the launch stream, so the kernels run back to back
    # with no host in the loop (a dispatch that records its own timing events runs
    # measurably slower, and a Python launch loop cannot keep up with the kernel).
    # Only the masks (the small output block) are kept; the bulk block of feature
    # rows and encodings is released after each launch, so the graph's pool hands
    # the same memory to the next launch, as the caching allocator does in the loop
    rmasks = []
    kern_ms = 0.0
    if R:
        args = pipe.launch_args(raws[W + K])
        eager = [int(sum(int(m.sum()) for m in pipe.launch(raws[i], args)["mask"]))
                 for i in range(W + K, min(W + K + 3, total))]
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(W + K, total):
                rmasks.append(tuple(pipe.launch(raws[i], args)["mask"]))
        graph.replay()  # first replay uploads the graph
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        kern_ms = e0.elapsed_time(e1)
        replayed = [int(sum(int(m.sum()) for m in ms)) for ms in rmasks[:len(eager)]]
        if replayed != eager:
            raise RuntimeError(f"graph replay disagrees with eager launches: {replayed} vs {eager}")
        del graph
        # the replays leave the ring where the timed region did: stream the window's
        # batches through it (untimed), so what follows sees the whole stream
        for i in range(W + K, total):
            pipe.prepare(raws[i])
            g.advance(raws[i].src, raws[i].dst, raws[i].time, raws[i].edge_feat)
        torch.cuda.synchronize()
    n_launch = max(R, 1)
    st = g.status()
    if any(st.values()):
        raise RuntimeError(f"device diagnostics: {st}")

    def algo_bytes(mask_list, first):
        qs = [int(sum(m.shape[0] for m in ms)) for ms in mask_list]
        vs = [int(sum(int(m.sum()) for m in ms)) for ms in mask_list]
        prs = [lens[first + j] if cfg.co_occurrence else 0 for j in range(len(mask_list))]
        return qs, vs, [bytes_per_batch(cfg, qs[j], vs[j], prs[j]) for j in range(len(mask_list))]

    rQs, rVs, rbyts = algo_bytes(rmasks, W + K)
    value = total_q / wall
    avg_launch_s = kern_ms / 1e3 / n_launch
    achieved = sum(rbyts) / n_launch / avg_launch_s / 1e9 if rbyts else 0.0
    log(f"timed {K} steps: wall {wall * 1e3:.1f} ms ({wall / K * 1e6:.1f} us/step); roofline window "
        f"{R} launches: {avg_launch_s * 1e6:.2f} us/launch, {achieved:.0f} GB/s, mean V/query "
        f"{sum(rVs) / max(sum(rQs), 1):.2f}")

    if a.copy_calibration_mib > 0:
        n = a.copy_calibration_mib << 20
        src_buf = torch.ones(n // 4, dtype=torch.float32, device=device)
        dst_buf = torch.empty_like(src_buf)
        for _ in range(3):
            dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        del src_buf, dst_buf

    ceilings = None
    if a.ceilings:
        ceilings = measure_ceilings(torch, device, int(sum(rbyts) / n_launch) if rbyts else 1 << 27, log)

    # HBM traffic per launch from the byte counters of a profiling run over the
    # same roofline window (profiles/<config>_recent_fused_pmc.json, one entry per
    # window); null when no profile covers this window
    traffic = None
    window = f"{W + K}..{total - 1}"
    pmc = ROOT / "profiles" / f"{cfg.name}_recent_fused_pmc.json"
    if pmc.exists():
        entry = json.loads(pmc.read_text()).get("windows", {}).get(window)
        if entry is not None:
            traffic = entry.get("traffic_bytes_per_launch")

    cpu = None
    if not a.no_cpu and total < avail:
        cpu = cpu_baseline(cfg, g, pipe, total, a.cpu_seconds, torch, log, num_batches(cfg))

    line = {
        "metric": METRIC, "value": value, "unit": "prepared queries/s", "n_gpus": 1,
        "steps": K, "warmup": W, "ms_per_step": wall * 1e3 / K, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int64/f64 ids+times, "
        + ("bf16" if cfg.feat_dtype == "bf16" else "f32") + " rows, f32 time-enc",
        "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.num_nodes} nodes, batch {cfg.batch}, "
                               f"K={cfg.k}, B={cfg.buffer_size}, d={cfg.feat_dim} {cfg.feat_dtype}, "
                               f"{cfg.queries_per_event} queries/event, d_t=100"
                               + (", co-occurrence" if cfg.co_occurrence else ""),
                   "batches_timed": f"{W}..{W + K - 1}", "events_per_batch": cfg.batch},
        "host_us_per_step": {"prepare": host_prep / K * 1e6, "advance": host_adv / K * 1e6},
        "timed_region": "prepare + advance of every batch, inputs resident in HBM, Python's "
                        "cyclic GC off, synchronised on both sides",
        "prepare_kernel": {"us_per_launch": avg_launch_s * 1e6, "launches": n_launch,
                           "batches": f"{W + K}..{total - 1}",
                           "queries_per_s": sum(rQs) / (kern_ms / 1e3) if kern_ms else None,
                           "mean_valid_per_query": sum(rVs) / max(sum(rQs), 1),
                           "bytes_per_launch": sum(rbyts) / n_launch},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "traffic_window": window if traffic is not None else None,
                     "kernel": "recent_fused",
                     "timing": f"HIP event pair around a graph replay of the {R} launches of "
                               f"batches {W + K}..{total - 1}"},
        "cpu_baseline": cpu,
    }
    if ceilings is not None:
        line["ceilings"] = ceilings
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
