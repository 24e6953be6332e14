"""The ring plan that DataPipeline.prepare runs inside its gather launch.

prepare(batch) plans the batch's ring update in the same launch as its gather;
advance() of the same tensors commits the plan, anything else discards it and
runs the whole update.  Every case compares the gathered neighbours and the ring
with the CPU oracle bit for bit: batches the fused plan covers, batches above
its size (planned by launches of their own), a second prepare before advance, a
query between plan and commit, advance with other tensors, and the
AsyncDataPipeline, whose plan is enqueued on its prefetch stream.
"""
import dataclasses

import numpy as np
import pytest
import torch

import stream_check as S
from oracle import spec as O
from tgengine_amd import AsyncDataPipeline, RawBatch
from tgengine_amd.synthetic import CONFIGS, gen_batch

pytestmark = pytest.mark.gpu

C1 = CONFIGS["c1"]


def _setup(cfg):
    fdt = np.uint16 if cfg.feat_dtype == "bf16" else np.float32
    g = S.make_graph(cfg)
    pipe = S.make_pipeline(cfg, g)
    ring = O.Ring.empty(cfg.num_nodes, cfg.buffer_size, cfg.feat_dim, fdt)
    return g, pipe, ring


def _advance_both(g, ring, rb, bt):
    g.advance(rb.src, rb.dst, rb.time, rb.edge_feat)
    O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], bt["feat"])


def _check_ring(g, ring, bt, where):
    S.compare_ring(g, ring, np.concatenate([bt["src"], bt["dst"]]), where)
    N = g.num_nodes
    assert int(g._ov_scratch[:N].abs().sum()) == 0, f"{where}: node counters not restored"


def _check_status(g):
    st = g.status()
    assert st == {"bad_event_nodes": 0, "key_collisions": 0, "bad_query_nodes": 0}, st


@pytest.mark.parametrize("batch", [200, 17000])  # fused plan / plan launched after the gather
def test_prepare_advance_plans_match_the_oracle(batch):
    cfg = dataclasses.replace(C1, batch=batch)
    g, pipe, ring = _setup(cfg)
    w = O.time_weights(100)
    for i in range(4):
        bt = gen_batch(cfg, i)
        rb = S.to_raw(cfg, bt)
        pb = pipe.prepare(rb)
        assert (g._plan is not None) == (i > 0)  # the ring exists from the first advance on
        S.compare_prepared(cfg, pb, bt, ring if i > 0 else None, w, f"batch {i}")
        _advance_both(g, ring, rb, bt)
        assert g._plan is None
        _check_ring(g, ring, bt, f"ring after {i}")
    _check_status(g)


def test_second_prepare_replans_and_queries_between_plan_and_commit():
    cfg = C1
    g, pipe, ring = _setup(cfg)
    w = O.time_weights(100)
    for i in range(5):
        bt = gen_batch(cfg, i)
        rb = S.to_raw(cfg, bt)
        pipe.prepare(rb)
        pb = pipe.prepare(rb)  # the first plan is dropped, this one is committed
        # a plain query sees the ring before this batch while the plan is pending
        nodes, qt = S.queries_of(bt)
        nd = g.recent(torch.from_numpy(nodes).cuda(), torch.from_numpy(qt).cuda(), cfg.k)
        ref = O.recent(nodes, qt, cfg.k, None, ring if i > 0 else None, cfg.feat_dim, np.float32)
        assert np.array_equal(nd.neighbor_ids.cpu().numpy(), ref.ids), f"batch {i}: recent ids"
        S.compare_prepared(cfg, pb, bt, ring if i > 0 else None, w, f"batch {i}")
        _advance_both(g, ring, rb, bt)
        _check_ring(g, ring, bt, f"ring after {i}")
    _check_status(g)


def test_advance_with_other_tensors_discards_the_plan():
    cfg = C1
    g, pipe, ring = _setup(cfg)
    for i in range(5):
        bt = gen_batch(cfg, i)
        rb = S.to_raw(cfg, bt)
        pipe.prepare(rb)
        if i % 2:
            # equal values in other tensors: the plan is dropped, the batch still applies
            g.advance(rb.src.clone(), rb.dst.clone(), rb.time.clone(), rb.edge_feat)
            O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], bt["feat"])
        else:
            _advance_both(g, ring, rb, bt)
        assert g._plan is None
        _check_ring(g, ring, bt, f"ring after {i}")
    _check_status(g)


def test_plan_updates_off_gives_the_same_ring():
    cfg = C1
    g, pipe, ring = _setup(cfg)
    pipe.plan_updates = False
    for i in range(4):
        bt = gen_batch(cfg, i)
        rb = S.to_raw(cfg, bt)
        pipe.prepare(rb)
        assert g._plan is None
        _advance_both(g, ring, rb, bt)
        _check_ring(g, ring, bt, f"ring after {i}")
    _check_status(g)


class _GivenNegatives:
    """Negative strategy returning the generator's negatives of each batch."""

    def __init__(self):
        self.queue = []

    def sample(self, src, dst, time, graph, edge_indices):
        return self.queue.pop(0)


def test_async_pipeline_plans_on_its_prefetch_stream():
    cfg = C1
    g = S.make_graph(cfg)
    neg = _GivenNegatives()
    spec = S.make_pipeline(cfg, g).spec
    ap = AsyncDataPipeline(spec, g, neg)
    ring = O.Ring.empty(cfg.num_nodes, cfg.buffer_size, cfg.feat_dim, np.float32)
    w = O.time_weights(100)
    bts = [gen_batch(cfg, i) for i in range(6)]
    raws = [S.to_raw(cfg, bt) for bt in bts]
    for i, (bt, rb) in enumerate(zip(bts, raws)):
        # odd batches are prefetched twice without a get() between: the first
        # prefetch is joined and dropped, its plan replaced by the second's
        for _ in range(1 + i % 2):
            neg.queue.append(rb.neg)
            ap.start_prefetch(RawBatch(src=rb.src, dst=rb.dst, time=rb.time, edge_feat=rb.edge_feat))
        rb2, pb = ap.get()
        assert not neg.queue
        S.compare_prepared(cfg, pb, bt, ring if i > 0 else None, w, f"async batch {i}")
        g.advance(rb2.src, rb2.dst, rb2.time, rb2.edge_feat)
        O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], bt["feat"])
        assert g._plan is None
        _check_ring(g, ring, bt, f"async ring after {i}")
    _check_status(g)


# spin length of the bounded delay kernels (GPU clock cycles; a few ms)
SPIN = 20_000_000


class _SlowNegatives(_GivenNegatives):
    """Hands out given negatives after a bounded spin kernel on the current
    stream, which inside the prefetch thread is the prefetch stream."""

    def sample(self, src, dst, time, graph, edge_indices):
        torch.cuda._sleep(SPIN)
        return self.queue.pop(0)


def test_async_pipeline_orders_its_streams_under_delays():
    """The prefetch protocol (reference pipeline/async_pipeline.py:85-139) with
    bounded delay kernels that make each ordering step necessary:

    * a spin on the caller's stream right before advance(i): the commit of batch
      i is queued behind it, so prepare(i+1) on the prefetch stream reads the
      ring before batch i lands unless start_prefetch makes the prefetch stream
      wait for the caller's stream (AsyncDataPipeline.start_prefetch) -- the
      neighbours of batch i+1 would then miss batch i's events;
    * a spin on the prefetch stream before prepare(i+1): its outputs are written
      late, so the caller's copies (``.cpu()`` on the caller's stream) and the
      caller's advance(i+1), whose commit reads the plan written on the prefetch
      stream, see unwritten memory unless get() makes the caller's stream wait
      for the prefetch stream.
    The plan handed over by get() (TemporalGraph._adopt_plan) only spares
    advance() a second wait on the prefetch stream: without it advance() orders
    itself after the plan's stream on its own (_order_after), so no delay can
    expose its absence; it is checked here by the plan living on the caller's
    stream after get()."""
    cfg = C1
    g = S.make_graph(cfg)
    neg = _SlowNegatives()
    spec = S.make_pipeline(cfg, g).spec
    ap = AsyncDataPipeline(spec, g, neg)
    ring = O.Ring.empty(cfg.num_nodes, cfg.buffer_size, cfg.feat_dim, np.float32)
    w = O.time_weights(100)
    bts = [gen_batch(cfg, i) for i in range(8)]
    raws = [S.to_raw(cfg, bt) for bt in bts]
    caller = torch.cuda.current_stream()
    neg.queue.append(raws[0].neg)
    ap.start_prefetch(RawBatch(src=raws[0].src, dst=raws[0].dst, time=raws[0].time,
                               edge_feat=raws[0].edge_feat))
    for i, bt in enumerate(bts):
        rb2, pb = ap.get()
        if g._plan is not None:
            assert g._plan.stream == caller.cuda_stream  # handed over to the caller's stream
        S.compare_prepared(cfg, pb, bt, ring if i > 0 else None, w, f"delayed async batch {i}")
        torch.cuda._sleep(SPIN)  # the commit of batch i is queued behind this spin
        g.advance(rb2.src, rb2.dst, rb2.time, rb2.edge_feat)
        O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], bt["feat"])
        if i + 1 < len(bts):
            nxt = raws[i + 1]
            neg.queue.append(nxt.neg)
            ap.start_prefetch(RawBatch(src=nxt.src, dst=nxt.dst, time=nxt.time, edge_feat=nxt.edge_feat))
    torch.cuda.synchronize()
    _check_ring(g, ring, bts[-1], "delayed async ring")
    _check_status(g)


def test_many_batch_sizes_stay_exact_without_per_shape_state():
    # 70 distinct batch sizes, then a size seen before: the event-major grouping
    # is computed in the kernel, so nothing is cached per batch shape
    cfg = CONFIGS["c2"]  # co-occurrence: queries grouped by event
    g, pipe, ring = _setup(cfg)
    w = O.time_weights(100)
    sizes = [100 + i for i in range(70)] + [100]
    for i, b in enumerate(sizes):
        bt = {k: v[:b] for k, v in gen_batch(cfg, i).items()}
        rb = S.to_raw(cfg, bt)
        pb = pipe.prepare(rb)
        S.compare_prepared(cfg, pb, bt, ring if i > 0 else None, w, f"batch {i} of {b} events")
        _advance_both(g, ring, rb, bt)
    assert not hasattr(pipe, "_plans")
    _check_ring(g, ring, bt, "ring after the last batch")
    _check_status(g)


@pytest.mark.parametrize("shape", ["singletons", "one_node", "pairs", "groups10"])
def test_fused_plan_batch_shapes(shape):
    """The plan as the gather launch's first workgroups, on 4,000-event batches
    whose nodes all have the same number of entries (consecutive ids), against the
    oracle's ring after every batch."""
    cfg = dataclasses.replace(CONFIGS["c3"], num_nodes=60_000)
    g, pipe, ring = _setup(cfg)
    rng = np.random.default_rng(40)
    b = 4000
    i = np.arange(b, dtype=np.int64)
    for j in range(4):
        base = 1000 + 9973 * j
        if shape == "singletons":
            src, dst = base + 2 * i, base + 2 * i + 1
        elif shape == "one_node":
            src, dst = np.full(b, base), np.full(b, base)
        elif shape == "pairs":
            src, dst = base + i, base + (i + 1) % b
        else:
            src, dst = base + i % 800, base + (i + 7) % 800
        bt = dict(gen_batch(cfg, j))
        bt["src"], bt["dst"] = src, dst
        bt["neg"] = rng.integers(0, cfg.num_nodes, b)
        rb = S.to_raw(cfg, bt)
        pipe.prepare(rb)
        assert (g._plan is not None) == (j > 0)
        _advance_both(g, ring, rb, bt)
        _check_ring(g, ring, bt, f"{shape}: ring after {j}")
    _check_status(g)

