"""Fused gather (tgx_recent) through TemporalGraph / DataPipeline against the oracle.

Covers the frozen-CSR path, the ring path and their merge, padding queries,
K from 1 to 256, B up to 64, both dt conventions with and without a bias, time
encodings of widths that are and are not multiples of 4, every co-occurrence
mode, edge ids, negatives of shape (b, n), neg_src, 2-hop queries, and the
restated known-answer tests of the reference suite (tests/test_core.py,
tests/test_triton_kernel.py, tests/test_cuda_kernels.py, tests/test_negatives.py).
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import spec as O
from tgengine_amd import DataPipeline, GatherSpec, NeighborSpec, RawBatch, TemporalGraph
from tgengine_amd.core import _lib
from tgengine_amd.pipeline import cosine_time_weights

pytestmark = pytest.mark.gpu

TE_ATOL = 1e-6


def cu(x, dt=None):
    t = torch.as_tensor(x)
    return (t.to(dt) if dt is not None else t).cuda()


# ------------------------------------------------------------- known answers
def test_core_basic_csr():
    """reference tests/test_core.py:15-37"""
    g = TemporalGraph(10, buffer_size=8, edge_feat_dim=4, device="cuda")
    g.advance(cu([0, 0, 0, 1, 1]), cu([1, 2, 3, 2, 3]),
              cu([1.0, 2.0, 3.0, 1.5, 2.5], torch.float64), torch.randn(5, 4).cuda())
    assert g.num_edges == 5
    r = g.recent(cu([0]), cu([4.0], torch.float64), k=3)
    assert r.neighbor_ids.shape == (1, 3) and r.mask.shape == (1, 3)
    assert bool(r.mask.all())


def test_core_time_filter():
    """reference tests/test_core.py:40-56"""
    g = TemporalGraph(5, buffer_size=4, edge_feat_dim=2, device="cuda")
    g.advance(cu([0, 0, 0]), cu([1, 2, 3]), cu([1.0, 5.0, 10.0], torch.float64), torch.randn(3, 2).cuda())
    r = g.recent(cu([0]), cu([6.0], torch.float64), k=3)
    assert int(r.mask.sum()) == 2
    assert r.neighbor_ids[0].tolist() == [-1, 1, 2]


def test_core_co_neighbors():
    """reference tests/test_core.py:59-76"""
    g = TemporalGraph(10, buffer_size=8, edge_feat_dim=2, device="cuda")
    g.advance(cu([0, 0, 1, 1]), cu([2, 3, 2, 3]), cu([1.0, 2.0, 1.5, 2.5], torch.float64),
              torch.randn(4, 2).cuda())
    co = g.co_neighbors(cu([0]), cu([1]), cu([10.0], torch.float64))
    assert co.shape == (1,) and co.dtype == torch.float32 and co.item() == 2.0


def test_core_snapshot_restore():
    """reference tests/test_core.py:79-106, plus the ring contents"""
    g = TemporalGraph(5, buffer_size=4, edge_feat_dim=2, device="cuda")
    g.freeze_csr()
    g.advance(cu([0, 1]), cu([1, 2]), cu([1.0, 2.0], torch.float64), torch.randn(2, 2).cuda())
    snap = g.snapshot()
    ids0 = g._ov_ids.clone()
    g.advance(cu([2]), cu([3]), cu([3.0], torch.float64), torch.randn(1, 2).cuda())
    assert g.num_edges == 3
    g.restore(snap)
    assert g.num_edges == 2
    assert torch.equal(g._ov_ids, ids0)


def test_snapshot_restore_keeps_edge_ids():
    g = TemporalGraph(5, buffer_size=4, edge_feat_dim=2, device="cuda", track_edge_ids=True)
    g.freeze_csr()
    g.advance(cu([0, 1]), cu([1, 2]), cu([1.0, 2.0], torch.float64), torch.randn(2, 2).cuda())
    snap = g.snapshot()
    eids0 = g._ov_eids.clone()
    g.advance(cu([1]), cu([0]), cu([3.0], torch.float64), torch.randn(1, 2).cuda())
    assert not torch.equal(g._ov_eids, eids0)
    g.restore(snap)
    assert torch.equal(g._ov_eids, eids0)
    # a snapshot without edge ids (the reference's four ring arrays) cannot restore them
    bare = dataclasses.replace(snap, overflow_eids=None)
    with pytest.raises(ValueError):
        g.restore(bare)
    assert torch.equal(g._ov_eids, eids0) and g.num_edges == 2


def test_async_ordering_ring_known_answer():
    """reference tests/test_async_pipeline.py:153-194 (ring path, synchronous form)"""
    g = TemporalGraph(10, buffer_size=8, edge_feat_dim=2, device="cuda")
    g.recent(cu([1]), cu([0.5], torch.float64), 8)  # first query freezes an empty CSR
    g.advance(cu([1]), cu([2]), cu([1.0], torch.float64), torch.randn(1, 2).cuda())
    r = g.recent(cu([1]), cu([2.0], torch.float64), 8)
    assert 2 in r.neighbor_ids[0].tolist()


def test_triton_time_filtering_and_padding_queries():
    """reference tests/test_triton_kernel.py:76-117"""
    g = TemporalGraph(10, edge_feat_dim=16, device="cuda")
    g.advance(torch.zeros(10, dtype=torch.long).cuda(), (torch.arange(1, 11) % 10).cuda(),
              (torch.arange(1, 11, dtype=torch.float64) * 0.1).cuda(), torch.randn(10, 16).cuda())
    g.freeze_csr()
    r = g.recent(cu([0]), cu([0.55], torch.float64), k=10)
    assert int(r.mask[0].sum()) == 5
    assert bool((r.timestamps[0][r.mask[0]] < 0.55).all())
    r = g.recent(cu([-1, -1, 5, 10 % 10]), cu([0.5] * 4, torch.float64), 8)
    assert (r.neighbor_ids[:2] == -1).all() and int(r.mask[:2].sum()) == 0


def test_cuda_co_neighbor_disjoint_and_self():
    """reference tests/test_cuda_kernels.py:225-263"""
    src = torch.cat([torch.zeros(10, dtype=torch.long), torch.full((10,), 11, dtype=torch.long)])
    dst = torch.cat([torch.arange(1, 11), torch.arange(12, 22)])
    g = TemporalGraph(30, edge_feat_dim=16, device="cuda")
    g.advance(src.cuda(), dst.cuda(), (torch.arange(20, dtype=torch.float64) * 0.01).cuda(),
              torch.randn(20, 16).cuda())
    g.freeze_csr()
    assert g.co_neighbors(cu([0]), cu([11]), cu([1.0], torch.float64), k=10).item() == 0.0
    g2 = TemporalGraph(20, edge_feat_dim=16, device="cuda")
    g2.advance(torch.zeros(5, dtype=torch.long).cuda(), torch.arange(1, 6).cuda(),
               (torch.arange(5, dtype=torch.float64) * 0.1).cuda(), torch.randn(5, 16).cuda())
    assert g2.co_neighbors(cu([0]), cu([0]), cu([1.0], torch.float64), k=10).item() == 5.0


def test_negatives_co_occur_fusion_matches_graph_method():
    """reference tests/test_negatives.py:127-157"""
    g = TemporalGraph(20, buffer_size=8, edge_feat_dim=4, device="cuda")
    g.advance(cu([0, 0, 1, 1, 2]), cu([5, 6, 5, 7, 8]), cu([1.0, 2.0, 1.5, 2.5, 3.0], torch.float64),
              torch.randn(5, 4).cuda())
    pipe = DataPipeline(GatherSpec(neighbors=NeighborSpec(k=8), co_occurrence=True), g)
    src, dst = cu([0, 0, 1]), cu([1, 2, 2])
    t = cu([10.0, 10.0, 10.0], torch.float64)
    pb = pipe.prepare(RawBatch(src=src, dst=dst, time=t, neg=cu([3, 3, 3])))
    direct = g.co_neighbors(src, dst, t, k=8)
    assert torch.equal(pb.co_occurrence, direct)
    fused2 = DataPipeline._co_occur_from_neighbors(pb.src_neighbors, pb.dst_neighbors)
    assert torch.equal(fused2, direct)
    assert pb.co_occurrence.dtype == torch.float32 and bool((pb.co_occurrence >= 0).all())


# ------------------------------------------------------------- random parity
def _build(seed, N, B, d, K, with_pre, with_ring, bf16=False, eids=False, n_pre=3, n_ring=4, b=60):
    rng = np.random.default_rng(seed)
    fdt = np.uint16 if bf16 else np.float32
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=B,
                      feat_dtype=torch.bfloat16 if bf16 else torch.float32, track_edge_ids=eids)
    events, eb, t = [], 0, 1000.0
    def batch():
        nonlocal t
        src = rng.integers(0, N, b)
        dst = rng.integers(0, N, b)
        hot = rng.random(b) < 0.3
        src = np.where(hot, 1, src)
        time = t + np.cumsum(rng.exponential(1.0, b) + 1e-3)
        t = float(time[-1])
        f = rng.standard_normal((b, d)).astype(np.float32)
        if bf16:
            from tgengine_amd.synthetic import f32_to_bf16_bits
            f = f32_to_bf16_bits(f)
        return src, dst, time, f
    def dev_feat(f):
        x = torch.from_numpy(f)
        return (x.view(torch.bfloat16) if bf16 else x).cuda()
    if with_pre:
        for _ in range(n_pre):
            s, d_, tm, f = batch()
            g.advance(cu(s), cu(d_), cu(tm), dev_feat(f))
            events.append((s, d_, tm, f, eb))
            eb += b
    g.freeze_csr()
    csr = O.csr_freeze(N, d, events, fdt) if with_pre else O.CSR.empty(N, d, fdt)
    ring = None
    if with_ring:
        ring = O.Ring.empty(N, B, d, fdt, with_eids=True)
        for _ in range(n_ring):
            s, d_, tm, f = batch()
            g.advance(cu(s), cu(d_), cu(tm), dev_feat(f))
            O.ring_advance(ring, s, d_, tm, f, eid_base=eb)
            eb += b
    return rng, g, csr, ring, t


@pytest.mark.parametrize("K", [20, 64])
def test_csr_window_search_sizes(K):
    """recent() on a frozen CSR whose windows hold 1, 64, 65, 4,097 and about 5,000
    entries (a 64-ary search of one to three rounds, probes clamped to the window's
    last entry), with tied times, queried before the window, at exact entry times
    around the 64-boundaries, between entries and after the window: ids, times,
    rows and masks bit for bit against the oracle."""
    rng = np.random.default_rng(K)
    N, d = 8, 4
    sizes = {0: 5003, 1: 65, 2: 64, 3: 4097, 4: 1}
    src = np.concatenate([np.full(c, u) for u, c in sizes.items()])
    rng.shuffle(src)
    E = len(src)
    dst = rng.integers(5, N, E)  # destinations outside the measured nodes 0..4
    time = np.cumsum(rng.integers(0, 3, E).astype(np.float64)) + 100.0  # steps of 0: tied times
    feat = rng.standard_normal((E, d)).astype(np.float32)
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=8)
    events = []
    for lo in range(0, E, 2048):
        hi = min(E, lo + 2048)
        g.advance(cu(src[lo:hi]), cu(dst[lo:hi]), cu(time[lo:hi]), cu(feat[lo:hi]))
        events.append((src[lo:hi], dst[lo:hi], time[lo:hi], feat[lo:hi], lo))
    g.freeze_csr()
    csr = O.csr_freeze(N, d, events)
    nodes, qts = [], []
    for u in sizes:
        ts = np.sort(time[src == u])
        picks = [ts[0] - 1.0, ts[-1] + 1.0, ts[-1], ts[0]]
        for i in (1, 62, 63, 64, 65, 127, 128, 4095, 4096, len(ts) // 2, len(ts) - 2):
            if 0 <= i < len(ts):
                picks += [ts[i], ts[i] + 0.5]
        nodes += [u] * len(picks)
        qts += picks
    nodes = np.array(nodes, np.int64)
    qts = np.array(qts, np.float64)
    r = g.recent(cu(nodes), cu(qts), K)
    o = O.recent(nodes, qts, K, csr, None, d)
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
    assert np.array_equal(r.edge_feats.cpu().numpy(), o.feats)


def _feats_np(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


@pytest.mark.parametrize("with_pre,with_ring,K,B,bf16", [
    (True, False, 5, 8, False), (True, False, 64, 8, False), (False, True, 20, 32, True),
    (True, True, 7, 6, False), (True, True, 256, 64, False), (True, True, 1, 3, True),
    (False, True, 100, 64, False)])
def test_recent_matches_oracle(with_pre, with_ring, K, B, bf16):
    N, d = 40, 12
    rng, g, csr, ring, tmax = _build(11, N, B, d, K, with_pre, with_ring, bf16, eids=True)
    Q = 500
    nodes = rng.integers(-1, N, Q)
    qt = rng.uniform(900.0, tmax + 10.0, Q)  # includes queries before ring entries
    r = g.recent(cu(nodes), cu(qt), K)
    o = O.recent(nodes, qt, K, csr, ring, d, np.uint16 if bf16 else np.float32)
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(_feats_np(r.edge_feats).view(np.uint8), o.feats.view(np.uint8))
    assert np.array_equal(r.edge_ids.cpu().numpy(), o.eids)


def _tied_graph(seed, N, B, d, n_pre, b_pre, n_ring, b_ring):
    """A frozen CSR whose windows exceed 512 entries and a full ring, with times on an
    integer grid so that entries tie: within a CSR window, within a ring and
    between the two."""
    rng = np.random.default_rng(seed)
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=B)
    events, eb, t = [], 0, 5000.0
    def batch(b):
        nonlocal t
        src, dst = rng.integers(0, N, b), rng.integers(0, N, b)
        time = t + np.sort(rng.integers(0, b // 4, b)).astype(np.float64)
        t = float(time[-1])
        return src, dst, time, rng.standard_normal((b, d)).astype(np.float32)
    for _ in range(n_pre):
        s_, d_, tm, f = batch(b_pre)
        g.advance(cu(s_), cu(d_), cu(tm), cu(f))
        events.append((s_, d_, tm, f, eb))
        eb += b_pre
    g.freeze_csr()
    csr = O.csr_freeze(N, d, events, np.float32)
    ring = O.Ring.empty(N, B, d, np.float32)
    t -= b_ring // 2  # the ring's first batch starts before the CSR's last entries
    for _ in range(n_ring):
        s_, d_, tm, f = batch(b_ring)
        g.advance(cu(s_), cu(d_), cu(tm), cu(f))
        O.ring_advance(ring, s_, d_, tm, f, eid_base=eb)
        eb += b_ring
    return rng, g, csr, ring, t


# K up to 512 (LastFM's pipeline shape: K=512, 2-d fp32 rows): CSR windows longer
# than K, a ring of 64 slots, ties inside and across them, queries before, inside
# and after the windows; every output against the oracle
@pytest.mark.parametrize("K,with_ring", [(512, True), (512, False), (300, True)])
def test_recent_large_k_matches_oracle(K, with_ring):
    rng, g, csr, ring, tmax = _tied_graph(51, 6, 64, 2, 5, 600, 3 if with_ring else 0, 200)
    Q = 300
    nodes = rng.integers(-1, 6, Q)
    qt = np.floor(rng.uniform(5000.0, tmax + 5.0, Q))  # on the grid: ties with entries
    r = g.recent(cu(nodes), cu(qt), K)
    o = O.recent(nodes, qt, K, csr, ring if with_ring else None, 2)
    assert int(o.mask.sum(1).max()) == K  # some windows are truncated to K
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(r.edge_feats.cpu().numpy(), o.feats)


@pytest.mark.parametrize("mode", ["freq", "dygformer"])
def test_prepare_k512_lastfm_shape(mode):
    """DataPipeline.prepare at K=512 on the CSR + ring, with time encodings and
    co-occurrence (ii) / (iii)."""
    rng, g, csr, ring, tmax = _tied_graph(52, 8, 64, 2, 6, 500, 3, 200)
    K, b = 512, 40
    spec = GatherSpec(neighbors=NeighborSpec(k=K), time_encoding=100, co_occurrence=True,
                      co_occurrence_mode=mode)
    pipe = DataPipeline(spec, g)
    src, dst, neg = rng.integers(0, 8, b), rng.integers(0, 8, b), rng.integers(0, 8, b)
    t = tmax + np.floor(rng.uniform(0.0, 3.0, b))
    pb = pipe.prepare(RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg)))
    nodes = np.concatenate([src, dst, neg])
    qt = np.concatenate([t, t, t])
    o = O.recent(nodes, qt, K, csr, ring, 2)
    groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
    assert np.array_equal(torch.cat([x.neighbor_ids for x in groups]).cpu().numpy(), o.ids)
    assert np.array_equal(torch.cat([x.timestamps for x in groups]).cpu().numpy().view(np.int64),
                          o.times.view(np.int64))
    assert np.array_equal(torch.cat([x.mask for x in groups]).cpu().numpy(), o.mask)
    assert np.array_equal(torch.cat([x.edge_feats for x in groups]).cpu().numpy(), o.feats)
    te = torch.cat([x.time_enc for x in groups]).cpu().numpy()
    exp = O.time_encode_exact(O.dt_dygformer(qt, o.times), O.time_weights(100), o.mask)
    assert np.max(np.abs(te - exp)) <= TE_ATOL
    a, c = o.ids[:b], o.ids[b:2 * b]
    if mode == "freq":
        ea, ec = O.co_occurrence_freq(a, c)
    else:
        ea, ec = O.co_dygformer(np.concatenate([src[:, None], a], 1), np.concatenate([dst[:, None], c], 1))
    ga, gc = pb.co_occurrence_freq
    assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gc.cpu().numpy(), ec)
    assert np.array_equal(pb.co_occurrence.cpu().numpy(), O.co_pair_count(a, o.mask[:b], c, o.mask[b:2 * b]))


def test_recent_bad_query_nodes_are_padding_and_flagged():
    rng, g, csr, ring, tmax = _build(12, 20, 4, 3, 4, True, True)
    r = g.recent(cu([0, 25, 3]), cu([tmax + 1] * 3, torch.float64), 4)
    assert (r.neighbor_ids[1] == -1).all() and not bool(r.mask[1].any())
    assert g.status()["bad_query_nodes"] == 1


@pytest.mark.parametrize("dt_mode,d_t,bias", [("dygformer", 100, False), ("tgn", 100, False),
                                              ("dygformer", 37, False), ("dygformer", 100, True),
                                              ("tgn", 6, True)])
def test_time_encoding_modes(dt_mode, d_t, bias):
    rng, g, csr, ring, tmax = _build(13, 30, 16, 8, 10, True, True)

    class Enc(torch.nn.Module):
        def __init__(self):
            super().__init__()
            w = cosine_time_weights(d_t)
            self.linear = torch.nn.Linear(1, d_t)
            with torch.no_grad():
                self.linear.weight.copy_(torch.from_numpy(w).reshape(d_t, 1))
                self.linear.bias.copy_(torch.linspace(-1.0, 1.0, d_t) if bias else torch.zeros(d_t))

    enc = Enc()
    spec = GatherSpec(neighbors=NeighborSpec(k=10), time_encoding=d_t, dt_mode=dt_mode)
    pipe = DataPipeline(spec, g, time_encoder=enc)
    b = 64
    src = rng.integers(0, 30, b)
    dst = rng.integers(0, 30, b)
    neg = rng.integers(0, 30, b)
    t = tmax + rng.uniform(0.0, 50.0, b)
    pb = pipe.prepare(RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg)))
    nodes = np.concatenate([src, dst, neg])
    qt = np.concatenate([t, t, t])
    o = O.recent(nodes, qt, 10, csr, ring, 8)
    dt = O.dt_dygformer(qt, o.times) if dt_mode == "dygformer" else O.dt_tgn(qt, o.times)
    w = enc.linear.weight.detach().reshape(-1).numpy()
    bv = enc.linear.bias.detach().numpy() if bias else None
    exp = O.time_encode_exact(dt, w, o.mask if dt_mode == "dygformer" else None, bv)
    got = torch.cat([pb.src_neighbors.time_enc, pb.dst_neighbors.time_enc,
                     pb.neg_neighbors.time_enc]).cpu().numpy()
    assert got.shape == (3 * b, 10, d_t)
    assert np.max(np.abs(got - exp)) <= TE_ATOL


def test_time_encoding_large_arguments():
    """|dt| up to 1e9 and beyond 2^40 (slow path) keep the 1e-6 bound."""
    g = TemporalGraph(4, edge_feat_dim=2, device="cuda", buffer_size=4)
    g.freeze_csr()
    times = np.array([1.0, 3.5e7, 7.1e8, 9.9e8])
    g.advance(cu([0, 0, 0, 0]), cu([1, 2, 3, 1]), cu(times), torch.zeros(4, 2).cuda())
    w = np.float32([1.0, 3.7e3, 1e-9, 1e4])
    spec = GatherSpec(neighbors=NeighborSpec(k=4, for_nodes=("src",)), time_encoding=4, dt_mode="tgn")

    class Enc(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.linear = torch.nn.Linear(1, 4)
            with torch.no_grad():
                self.linear.weight.copy_(torch.from_numpy(w).reshape(4, 1))
                self.linear.bias.zero_()

    pipe = DataPipeline(spec, g, time_encoder=Enc())
    qt = np.array([2.0e9, 1.0e9 + 0.25])
    pb = pipe.prepare(RawBatch(src=cu([0, 0]), dst=cu([1, 1]), time=cu(qt)))
    r = g.recent(cu([0, 0]), cu(qt), 4)
    dt = O.dt_tgn(qt, r.timestamps.cpu().numpy())
    exp = O.time_encode_exact(dt, w)
    assert np.max(np.abs(pb.src_neighbors.time_enc.cpu().numpy() - exp)) <= TE_ATOL
    assert (np.abs(O.time_args(dt, w)) >= 2 ** 40).any()


def test_time_encoding_caller_bounds():
    """The fixed-weight pipeline passes its weights' bound (max|w| = 1) to the
    kernel: arguments past 2^29 still take the full-range reduction (1e-6 bound),
    and the same launch without bounds (every element on the full-range path)
    gives the same bits."""
    g = TemporalGraph(4, edge_feat_dim=2, device="cuda", buffer_size=4)
    g.freeze_csr()
    times = np.array([1.0, 3.5e7, 7.1e8, 9.9e8])
    g.advance(cu([0, 0, 0, 0]), cu([1, 2, 3, 1]), cu(times), torch.zeros(4, 2).cuda())
    spec = GatherSpec(neighbors=NeighborSpec(k=4, for_nodes=("src",)), time_encoding=4, dt_mode="tgn")
    pipe = DataPipeline(spec, g)
    qt = np.array([2.0e9, 1.0e9 + 0.25, 5.0e8, 3.6e7])
    src = cu([0, 0, 0, 0])
    pb = pipe.prepare(RawBatch(src=src, dst=cu([1, 1, 1, 1]), time=cu(qt)))
    r = g.recent(src, cu(qt), 4)
    dt = O.dt_tgn(qt, r.timestamps.cpu().numpy())
    w = cosine_time_weights(4)
    args = np.abs(O.time_args(dt, w))
    assert (args >= 2 ** 29).any() and (args[np.isfinite(args)] < 2 ** 29).any()
    exp = O.time_encode_exact(dt, w)
    assert np.max(np.abs(pb.src_neighbors.time_enc.cpu().numpy() - exp)) <= TE_ATOL
    wt = torch.from_numpy(w).cuda()
    groups = [(src, cu(qt), 1)]
    with_b = g._query(None, None, 4, groups=groups, d_t=4, te_w=wt, dt_mode=_lib.TGX_DT_TGN,
                      te_bounds=(1.0, 0.0))["te"][0]
    without = g._query(None, None, 4, groups=groups, d_t=4, te_w=wt, dt_mode=_lib.TGX_DT_TGN)["te"][0]
    assert torch.equal(with_b.view(torch.int32), without.view(torch.int32))
    assert np.max(np.abs(with_b.cpu().numpy() - exp)) <= TE_ATOL
    # with a bias: bounds (max|w|, max|b|) against none, and the oracle
    bias = np.float32([0.5, -3.0e8, 2.0, -0.25])
    bt = torch.from_numpy(bias).cuda()
    bounds = (float(np.abs(w).max()), float(np.abs(bias).max()))
    with_b = g._query(None, None, 4, groups=groups, d_t=4, te_w=wt, te_b=bt, dt_mode=_lib.TGX_DT_TGN,
                      te_bounds=bounds)["te"][0]
    without = g._query(None, None, 4, groups=groups, d_t=4, te_w=wt, te_b=bt,
                       dt_mode=_lib.TGX_DT_TGN)["te"][0]
    assert torch.equal(with_b.view(torch.int32), without.view(torch.int32))
    exp_b = O.time_encode_exact(dt, w, None, bias)
    assert np.max(np.abs(with_b.cpu().numpy() - exp_b)) <= TE_ATOL


# k <= 32 counts both sides in one pass, k > 32 side by side; 90 events with 1 or 3
# negatives each put the (src, dst) pair in the event's workgroup and tile the
# negatives after them
@pytest.mark.parametrize("mode,k,n_neg", [("freq", 12, 1), ("dygformer", 12, 1), ("freq", 40, 3),
                                          ("dygformer", 40, 3)])
def test_co_occurrence_modes(mode, k, n_neg):
    rng, g, csr, ring, tmax = _build(14, 12, 16, 4, 12, True, True, b=80)
    spec = GatherSpec(neighbors=NeighborSpec(k=k), co_occurrence=True, co_occurrence_mode=mode)
    pipe = DataPipeline(spec, g)
    b = 90
    src = rng.integers(-1, 12, b)
    dst = np.where(rng.random(b) < 0.2, src, rng.integers(0, 12, b))
    neg = rng.integers(0, 12, (b, n_neg)) if n_neg > 1 else rng.integers(0, 12, b)
    t = tmax + rng.uniform(0.0, 5.0, b)
    pb = pipe.prepare(RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg)))
    a = pb.src_neighbors.neighbor_ids.cpu().numpy()
    c = pb.dst_neighbors.neighbor_ids.cpu().numpy()
    o = O.recent(np.concatenate([src, dst]), np.concatenate([t, t]), k, csr, ring, 4)
    on = O.recent(neg.reshape(-1), np.repeat(t, n_neg), k, csr, ring, 4)
    assert np.array_equal(pb.neg_neighbors.neighbor_ids.cpu().numpy().reshape(-1, k), on.ids)
    assert np.array_equal(np.concatenate([a, c]), o.ids)
    if mode == "freq":
        ea, ec = O.co_occurrence_freq(a, c)
    else:
        A = np.concatenate([src[:, None], a], 1)
        C = np.concatenate([dst[:, None], c], 1)
        ea, ec = O.co_dygformer(A, C)
    ga, gc = pb.co_occurrence_freq
    assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gc.cpu().numpy(), ec)
    pair = O.co_pair_count(a, pb.src_neighbors.mask.cpu().numpy(), c, pb.dst_neighbors.mask.cpu().numpy())
    assert np.array_equal(pb.co_occurrence.cpu().numpy(), pair)


# more queries per event than a workgroup takes (TGX_MAX_GROUP = 8): the (src, dst)
# pair shares the event's workgroup and the negatives are tiled after them, for
# launches below and above 4,096 queries; prepare(), launch() and the 2-hop prepare
@pytest.mark.parametrize("n_neg,b,neg_src", [(7, 1000, False), (10, 300, False), (10, 1000, True),
                                             (6, 700, True)])
def test_co_occurrence_with_many_negatives(n_neg, b, neg_src):
    rng, g, csr, ring, tmax = _build(31, 40, 16, 4, 12, True, True, b=80)
    k = 12
    spec = GatherSpec(neighbors=NeighborSpec(k=k), co_occurrence=True, time_encoding=8)
    pipe = DataPipeline(spec, g)
    src = rng.integers(0, 40, b)
    dst = np.where(rng.random(b) < 0.2, src, rng.integers(0, 40, b))
    neg = rng.integers(0, 40, (b, n_neg))
    ns = rng.integers(0, 40, b) if neg_src else None
    t = tmax + rng.uniform(0.0, 5.0, b)
    rb = RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg),
                  neg_src=cu(ns) if neg_src else None)
    nodes = np.concatenate([src, dst, neg.reshape(-1)] + ([ns] if neg_src else []))
    qt = np.concatenate([t, t, np.repeat(t, n_neg)] + ([t] if neg_src else []))
    o = O.recent(nodes, qt, k, csr, ring, 4)
    a, c = o.ids[:b], o.ids[b:2 * b]
    ea, ec = O.co_occurrence_freq(a, c)
    pair = O.co_pair_count(a, o.mask[:b], c, o.mask[b:2 * b])
    pb = pipe.prepare(rb)
    groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors] + ([pb.neg_src_neighbors] if neg_src else [])
    assert np.array_equal(torch.cat([x.neighbor_ids for x in groups]).cpu().numpy(), o.ids)
    assert np.array_equal(torch.cat([x.mask for x in groups]).cpu().numpy(), o.mask)
    te = torch.cat([x.time_enc for x in groups]).cpu().numpy()
    assert np.max(np.abs(te - O.time_encode_exact(O.dt_dygformer(qt, o.times), O.time_weights(8), o.mask))) <= TE_ATOL
    ga, gc = pb.co_occurrence_freq
    assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gc.cpu().numpy(), ec)
    assert np.array_equal(pb.co_occurrence.cpu().numpy(), pair)
    # the raw launch of prepare() and the 2-hop prepare take the same layout
    out = pipe.launch(rb)
    assert np.array_equal(torch.cat(out["ids"]).cpu().numpy(), o.ids)
    assert np.array_equal(out["co_a"].cpu().numpy(), ea) and np.array_equal(out["co_c"].cpu().numpy(), ec)
    spec2 = GatherSpec(neighbors=NeighborSpec(k=k, k2=3), co_occurrence=True)
    pb2 = DataPipeline(spec2, g).prepare(rb)
    ga2, gc2 = pb2.co_occurrence_freq
    assert np.array_equal(ga2.cpu().numpy(), ea) and np.array_equal(gc2.cpu().numpy(), ec)
    assert np.array_equal(pb2.co_occurrence.cpu().numpy(), pair)


def test_standalone_co_occurrence_rows():
    rng = np.random.default_rng(15)
    a = rng.integers(-1, 9, (33, 70)).astype(np.int32)
    c = rng.integers(-1, 9, (33, 70)).astype(np.int32)
    from tgengine_amd.core import NeighborData
    z = torch.zeros(33, 70, dtype=torch.float64).cuda()
    nd_a = NeighborData(cu(a), z, torch.zeros(33, 70, 1).cuda(), cu(a != -1))
    nd_c = NeighborData(cu(c), z, torch.zeros(33, 70, 1).cuda(), cu(c != -1))
    got = DataPipeline._co_occur_from_neighbors(nd_a, nd_c).cpu().numpy()
    assert np.array_equal(got, O.co_pair_count(a, a != -1, c, c != -1))


def test_standalone_co_occurrence_uses_the_masks():
    # masked positions hold ordinary ids (not -1): the reference pair count reads
    # the masks (pipeline/__init__.py:206-219), so these must not count
    import ctypes
    from tgengine_amd.core import _lib
    rng = np.random.default_rng(16)
    P, K = 41, 37
    a = rng.integers(-1, 7, (P, K)).astype(np.int32)
    c = rng.integers(-1, 7, (P, K)).astype(np.int32)
    am = rng.random((P, K)) < 0.7
    cm = rng.random((P, K)) < 0.6
    from tgengine_amd.core import NeighborData
    z = torch.zeros(P, K, dtype=torch.float64).cuda()
    got = DataPipeline._co_occur_from_neighbors(NeighborData(cu(a), z, z, cu(am)),
                                                NeighborData(cu(c), z, z, cu(cm))).cpu().numpy()
    assert np.array_equal(got, O.co_pair_count(a, am, c, cm))
    # per-position counts through the C ABI, with and without masks
    ga, gc = cu(a), cu(c)
    gam, gcm = cu(am.astype(np.uint8)), cu(cm.astype(np.uint8))
    for masks, (ea, ec) in (((gam.data_ptr(), gcm.data_ptr()), O.co_occurrence_freq_masked(a, am, c, cm)),
                            ((None, None), O.co_occurrence_freq(a, c))):
        a_cnt = torch.empty((P, K, 2), dtype=torch.int32, device="cuda")
        c_cnt = torch.empty((P, K, 2), dtype=torch.int32, device="cuda")
        pair = torch.empty(P, dtype=torch.float32, device="cuda")
        rc = _lib.lib().tgx_co_occurrence(ga.data_ptr(), gc.data_ptr(), masks[0], masks[1], P, K,
                                          a_cnt.data_ptr(), c_cnt.data_ptr(), pair.data_ptr(),
                                          torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "tgx_co_occurrence")
        assert np.array_equal(a_cnt.cpu().numpy(), ea) and np.array_equal(c_cnt.cpu().numpy(), ec)


def test_pipeline_negatives_2d_and_neg_src():
    rng, g, csr, ring, tmax = _build(16, 25, 8, 6, 6, False, True, eids=True)
    spec = GatherSpec(neighbors=NeighborSpec(k=6), time_encoding=8, edge_ids=True)
    pipe = DataPipeline(spec, g)
    b = 40
    src, dst = rng.integers(0, 25, b), rng.integers(0, 25, b)
    neg = rng.integers(0, 25, (b, 5))
    neg_src = rng.integers(0, 25, b)
    t = tmax + rng.uniform(0.0, 3.0, b)
    pb = pipe.prepare(RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg), neg_src=cu(neg_src)))
    assert pb.neg_neighbors.neighbor_ids.shape == (5 * b, 6)
    nodes = np.concatenate([src, dst, neg.reshape(-1), neg_src])
    qt = np.concatenate([t, t, np.repeat(t, 5), t])
    o = O.recent(nodes, qt, 6, None, ring, 6)
    got = torch.cat([pb.src_neighbors.neighbor_ids, pb.dst_neighbors.neighbor_ids,
                     pb.neg_neighbors.neighbor_ids, pb.neg_src_neighbors.neighbor_ids]).cpu().numpy()
    assert np.array_equal(got, o.ids)
    eids = torch.cat([pb.src_neighbors.edge_ids, pb.dst_neighbors.edge_ids,
                      pb.neg_neighbors.edge_ids, pb.neg_src_neighbors.edge_ids]).cpu().numpy()
    assert np.array_equal(eids, o.eids)
    te = torch.cat([pb.src_neighbors.time_enc, pb.dst_neighbors.time_enc,
                    pb.neg_neighbors.time_enc, pb.neg_src_neighbors.time_enc]).cpu().numpy()
    exp = O.time_encode_exact(O.dt_dygformer(qt, o.times), O.time_weights(8), o.mask)
    assert np.max(np.abs(te - exp)) <= TE_ATOL


@pytest.mark.parametrize("with_pre,with_ring,bf16", [(True, True, False), (False, True, True),
                                                   (True, False, False)])
def test_recent_2hop_matches_oracle_composition(with_pre, with_ring, bf16):
    """hop 2 = recent() of every hop-1 slot's (id, time), padding under invalid hop-1
    slots (reference temporal_graph.py:453-472): ids, times, rows and masks of both
    hops bit-exact, padding query ids (< 0) included, no status counts."""
    N, d = 15, 3
    rng, g, csr, ring, tmax = _build(17, N, 8, d, 5, with_pre, with_ring, bf16)
    fdt = np.uint16 if bf16 else np.float32
    Q = 40
    nodes = rng.integers(-1, N, Q)
    qt = rng.uniform(tmax - 40.0, tmax + 1.0, Q)
    r = g.recent_2hop(cu(nodes), cu(qt), 5, 4)
    h1 = O.recent(nodes, qt, 5, csr, ring, d, fdt)
    h2 = O.recent(h1.ids.reshape(-1).astype(np.int64), h1.times.reshape(-1), 4, csr, ring, d, fdt)
    m2 = h2.mask.reshape(Q, 5, 4) & h1.mask[:, :, None]
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), h1.ids)
    assert np.array_equal(r.mask.cpu().numpy(), h1.mask)
    assert np.array_equal(r.hop2_mask.cpu().numpy(), m2)
    assert np.array_equal(r.hop2_ids.cpu().numpy(), np.where(m2, h2.ids.reshape(Q, 5, 4), -1))
    assert np.array_equal(r.hop2_times.cpu().numpy().view(np.int64),
                          np.where(m2, h2.times.reshape(Q, 5, 4), 0.0).view(np.int64))
    f2 = np.where(m2[..., None], h2.feats.reshape(Q, 5, 4, d), np.zeros((), fdt))
    assert np.array_equal(_feats_np(r.hop2_feats).view(np.uint8), f2.view(np.uint8))
    assert g.status() == {"bad_event_nodes": 0, "key_collisions": 0, "bad_query_nodes": 0}
    pipe = DataPipeline(GatherSpec(neighbors=NeighborSpec(k=5, k2=4)), g)
    nn = np.clip(nodes, 0, None)
    pb = pipe.prepare(RawBatch(src=cu(nn[:10]), dst=cu(nn[10:20]), time=cu(qt[:10]),
                               neg=cu(nn[20:30])))
    assert pb.src_neighbors.hop2_ids.shape == (10, 5, 4)


def test_int32_query_nodes_and_validity_mask():
    """A query group of int32 ids gives what int64 ids give; a False in its validity
    array makes that query padding only, with no bad-query count even for an
    out-of-range id."""
    rng, g, csr, ring, tmax = _build(18, 20, 8, 4, 6, True, True)
    Q = 64
    nodes = rng.integers(0, 20, Q)
    qt = rng.uniform(tmax - 30.0, tmax + 1.0, Q)
    valid = rng.random(Q) < 0.6
    n32 = nodes.astype(np.int32)
    n32[~valid & (np.arange(Q) % 2 == 0)] = 1000  # out of range, but masked
    ref = g._query(cu(nodes), cu(qt), 6)
    got = g._query(None, None, 6, groups=[(cu(n32), cu(qt), 1, cu(valid))])
    v = valid[:, None]
    for key, pad in (("ids", -1), ("times", 0.0), ("mask", False)):
        a = got[key][0].cpu().numpy()
        b = ref[key][0].cpu().numpy()
        assert np.array_equal(a, np.where(v, b, pad)), key
    fa, fb = got["feats"][0].cpu().numpy(), ref["feats"][0].cpu().numpy()
    assert np.array_equal(fa, np.where(v[..., None], fb, 0.0))
    assert g.status()["bad_query_nodes"] == 0


def test_edge_ids_need_a_tracking_graph():
    g = TemporalGraph(5, edge_feat_dim=2, device="cuda")
    pipe = DataPipeline(GatherSpec(neighbors=NeighborSpec(k=2), edge_ids=True), g)
    with pytest.raises(ValueError, match="track_edge_ids"):
        pipe.prepare(RawBatch(src=cu([0]), dst=cu([1]), time=cu([1.0], torch.float64), neg=cu([2])))


def test_from_dataset_and_dtype_checks():
    src = torch.randint(0, 50, (3000,))
    dst = torch.randint(0, 50, (3000,))
    t = torch.sort(torch.rand(3000, dtype=torch.float64))[0]
    f = torch.randn(3000, 7)
    g = TemporalGraph.from_dataset(src, dst, t, f, 50, device="cuda")
    assert g.num_edges == 3000 and g._frozen
    g2 = TemporalGraph(50, edge_feat_dim=7, device="cuda")
    g2.freeze_csr()
    with pytest.raises(RuntimeError, match="dtypes match"):
        g2.advance(cu([1]), cu([2]), cu([1.0], torch.float64), torch.randn(1, 7).bfloat16().cuda())
