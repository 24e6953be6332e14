"""recent() and DataPipeline.prepare on a frozen CSR through the ring-less
kernels at K <= 64: csr_window (more than 2,048 queries, each taking one
wavefront, rows of at most 64 bytes or none: 64 / Bp queries per wavefront) and
csr_split (the other launches: queries split over several wavefronts, or rows of
any width through memory).  Both answer a query from the window's last K entries
when it comes after the whole window, else from a search.

Windows of 0 to thousands of entries with tied times; queries before, inside, at
and after them, NaN query times, padding (-1) and out-of-range nodes, a validity
mask (the 2-hop's second hop), edge ids and time encodings in both dt modes.
Ids, times, masks, rows and edge ids bit for bit against the oracle; encodings
within 1e-6.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import spec as O
from tgengine_amd import DataPipeline, GatherSpec, NeighborSpec, RawBatch, TemporalGraph
from tgengine_amd.core import _lib
from tgengine_amd.pipeline import cosine_time_weights
from tgengine_amd.synthetic import f32_to_bf16_bits

pytestmark = pytest.mark.gpu

TE_ATOL = 1e-6


def cu(x):
    return torch.as_tensor(x).cuda()


def _stream(seed, N, d, bf16, E=24000, batch=4000):
    """A frozen CSR of E events on an integer time grid (ties) whose sources follow
    a Zipf law and whose destinations are the lower half of the nodes: windows of
    thousands of entries, and in the upper half windows of a few or none."""
    rng = np.random.default_rng(seed)
    fdt = np.uint16 if bf16 else np.float32
    src = np.minimum(rng.zipf(1.4, E) - 1, N - 1).astype(np.int64)
    dst = rng.integers(0, N // 2, E)
    time = 100.0 + np.cumsum(rng.integers(0, 3, E)).astype(np.float64)
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=8,
                      feat_dtype=torch.bfloat16 if bf16 else torch.float32, track_edge_ids=True)
    events = []
    for lo in range(0, E, batch):
        hi = min(E, lo + batch)
        f = rng.standard_normal((hi - lo, d)).astype(np.float32)
        if bf16:
            f = f32_to_bf16_bits(f)
        ft = torch.from_numpy(f)
        g.advance(cu(src[lo:hi]), cu(dst[lo:hi]), cu(time[lo:hi]),
                  (ft.view(torch.bfloat16) if bf16 else ft).cuda())
        events.append((src[lo:hi], dst[lo:hi], time[lo:hi], f, lo))
    g.freeze_csr()
    return rng, g, O.csr_freeze(N, d, events, fdt), float(time[-1]), fdt


def _queries(rng, N, Q, tmax):
    """Half after every window (the usual case once the CSR is frozen), the rest
    on the grid (exact ties), between grid points, before the stream and NaN."""
    nodes = np.minimum(rng.zipf(1.3, Q) - 1, N - 1)
    nodes = np.where(rng.random(Q) < 0.3, rng.integers(0, N, Q), nodes)
    nodes[rng.random(Q) < 0.03] = -1
    kind = rng.random(Q)
    qt = tmax + 1.0 + np.floor(rng.uniform(0.0, 3.0, Q))
    inside = np.floor(rng.uniform(95.0, tmax + 2.0, Q))
    qt = np.where(kind < 0.5, qt, inside)
    qt = np.where((kind >= 0.8) & (kind < 0.93), inside + 0.5, qt)
    qt = np.where((kind >= 0.93) & (kind < 0.96), 50.0, qt)
    qt[kind >= 0.96] = np.nan
    return nodes.astype(np.int64), qt


def _feats_u8(t):
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.cpu().numpy().view(np.uint8)


def _shape_m(g, Q, K, d_t=0):
    """Queries per wavefront of the launch recent() makes (csr_window packs
    64 / Bp of them; recent_fused's ring-less copy takes one)."""
    csr = g._csr()
    a = _lib.TgxRecentArgs(k=K, group=4, num_queries=Q, nodes=8, times=8, out_ids=8, out_times=8,
                           out_mask=8, out_feats=16 if g.edge_feat_dim > 0 else 0, d_t=d_t,
                           te_w=16 if d_t else 0, out_te=16 if d_t else 0)
    out = (ctypes.c_int64 * 8)()
    assert _lib.lib().tgx_recent_launch_shape(None, ctypes.byref(csr), ctypes.byref(a), out) == 0
    return out[3], out[4]


@pytest.mark.parametrize("d,bf16,K", [(4, False, 1), (16, True, 20), (12, False, 33),
                                      (16, False, 64), (16, True, 16), (8, True, 17)])
def test_csr_window_matches_oracle(d, bf16, K):
    N, Q = 400, 6000
    rng, g, csr, tmax, fdt = _stream(30 + K, N, d, bf16)
    nodes, qt = _queries(rng, N, Q, tmax)
    Bp = max(16, 1 << (K - 1).bit_length())
    assert _shape_m(g, Q, K) == (64 // Bp, 1)
    r = g.recent(cu(nodes), cu(qt), K)
    o = O.recent(nodes, qt, K, csr, None, d, fdt)
    lens = np.diff(csr.offsets)
    assert lens.max() > 2000 and (lens[lens > 0] <= K).any() and (lens == 0).any()
    assert o.mask.all(1).any() and (~o.mask).all(1).any()
    assert K == 1 or (o.mask.any(1) & ~o.mask.all(1)).any()  # rows with pads and entries
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(_feats_u8(r.edge_feats), o.feats.view(np.uint8))
    assert np.array_equal(r.edge_ids.cpu().numpy(), o.eids)
    assert g.status()["bad_query_nodes"] == 0


def test_csr_window_bad_nodes_are_padding_and_flagged():
    N, Q, K = 300, 3000, 20
    rng, g, csr, tmax, fdt = _stream(41, N, 16, True)
    nodes, qt = _queries(rng, N, Q, tmax)
    bad = rng.random(Q) < 0.01
    nodes[bad] = N + rng.integers(0, 5, int(bad.sum()))
    r = g.recent(cu(nodes), cu(qt), K)
    o = O.recent(np.where(bad, -1, nodes), qt, K, csr, None, 16, fdt)
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(_feats_u8(r.edge_feats), o.feats.view(np.uint8))
    assert g.status()["bad_query_nodes"] == int(bad.sum())


def test_csr_window_2hop_validity_mask():
    """hop 1 (3,000 queries, k1 = 20) and hop 2 (60,000 queries under hop 1's
    mask, k2 = 16) both through csr_window, against the oracle's composition."""
    N, Q, k1, k2, d = 400, 3000, 20, 16, 16
    rng, g, csr, tmax, fdt = _stream(42, N, d, True)
    nodes, qt = _queries(rng, N, Q, tmax)
    assert _shape_m(g, Q, k1)[0] == 2 and _shape_m(g, Q * k1, k2)[0] == 4
    r = g.recent_2hop(cu(nodes), cu(qt), k1, k2)
    h1 = O.recent(nodes, qt, k1, csr, None, d, fdt)
    h2 = O.recent(h1.ids.reshape(-1).astype(np.int64), h1.times.reshape(-1), k2, csr, None, d, fdt)
    m2 = h2.mask.reshape(Q, k1, k2) & h1.mask[:, :, None]
    assert m2.any() and not m2.all()
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), h1.ids)
    assert np.array_equal(r.mask.cpu().numpy(), h1.mask)
    assert np.array_equal(r.hop2_mask.cpu().numpy(), m2)
    assert np.array_equal(r.hop2_ids.cpu().numpy(), np.where(m2, h2.ids.reshape(Q, k1, k2), -1))
    assert np.array_equal(r.hop2_times.cpu().numpy().view(np.int64),
                          np.where(m2, h2.times.reshape(Q, k1, k2), 0.0).view(np.int64))
    f2 = np.where(m2[..., None], h2.feats.reshape(Q, k1, k2, d), np.zeros((), fdt))
    assert np.array_equal(_feats_u8(r.hop2_feats), f2.view(np.uint8))
    assert g.status()["bad_query_nodes"] == 0


@pytest.mark.parametrize("dt_mode,d_t,K", [("dygformer", 100, 16), ("tgn", 100, 16),
                                           ("dygformer", 37, 20), ("tgn", 8, 64)])
def test_csr_window_prepare_time_encoding(dt_mode, d_t, K):
    """DataPipeline.prepare on the frozen CSR (no advance, as the Engine runs its
    evaluation): 1,000 events, 3,000 queries in three query groups."""
    N, b, d = 400, 1000, 16
    rng, g, csr, tmax, fdt = _stream(43, N, d, False)
    spec = GatherSpec(neighbors=NeighborSpec(k=K), time_encoding=d_t, dt_mode=dt_mode)
    pipe = DataPipeline(spec, g)
    nodes, qt = _queries(rng, N, 3 * b, tmax)
    src, dst, neg = np.maximum(nodes[:b], 0), np.maximum(nodes[b:2 * b], 0), np.maximum(nodes[2 * b:], 0)
    t = np.where(np.isnan(qt[:b]), tmax + 1.0, qt[:b])
    assert _shape_m(g, 3 * b, K, d_t)[1] == 1  # one wave per query: the csr_window shape
    pb = pipe.prepare(RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg)))
    allq = np.concatenate([src, dst, neg])
    qts = np.concatenate([t, t, t])
    o = O.recent(allq, qts, K, csr, None, d, fdt)
    groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
    assert np.array_equal(torch.cat([x.neighbor_ids for x in groups]).cpu().numpy(), o.ids)
    assert np.array_equal(torch.cat([x.timestamps for x in groups]).cpu().numpy().view(np.int64),
                          o.times.view(np.int64))
    assert np.array_equal(torch.cat([x.mask for x in groups]).cpu().numpy(), o.mask)
    assert np.array_equal(torch.cat([x.edge_feats for x in groups]).cpu().numpy(), o.feats)
    dt = O.dt_dygformer(qts, o.times) if dt_mode == "dygformer" else O.dt_tgn(qts, o.times)
    exp = O.time_encode_exact(dt, cosine_time_weights(d_t), o.mask if dt_mode == "dygformer" else None)
    got = torch.cat([x.time_enc for x in groups]).cpu().numpy()
    assert got.shape == (3 * b, K, d_t)
    assert np.max(np.abs(got - exp)) <= TE_ATOL


def test_csr_max_time_is_recorded_and_only_a_hint():
    """freeze_csr records the largest non-NaN entry time in the CSR struct; the
    gather only uses it to decide whether a query may fall inside a window (and
    to issue its search's first round early), so any value gives the same
    answers: -inf (no query probes ahead), +inf (every query over a long window
    does) and the recorded one."""
    N, Q, K, d = 300, 4000, 20, 16
    rng, g, csr, tmax, fdt = _stream(44, N, d, True)
    assert g._csr().max_time == tmax == np.nanmax(csr.times)
    nodes, qt = _queries(rng, N, Q, tmax)
    o = O.recent(nodes, qt, K, csr, None, d, fdt)
    for hint in (float("-inf"), float("inf"), tmax):
        g._csr().max_time = hint
        r = g.recent(cu(nodes), cu(qt), K)
        assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids), hint
        assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64)), hint
        assert np.array_equal(r.mask.cpu().numpy(), o.mask), hint
        assert np.array_equal(_feats_u8(r.edge_feats), o.feats.view(np.uint8)), hint


@pytest.mark.parametrize("d,bf16,K,dt_mode", [(172, False, 32, "dygformer"), (172, False, 64, "tgn"),
                                              (16, True, 20, "dygformer"), (2, False, 512, "dygformer"),
                                              (2, False, 100, "tgn")])
def test_csr_split_prepare_engine_shape(d, bf16, K, dt_mode):
    """DataPipeline.prepare of 200-event batches on the frozen CSR, as the Engine
    runs it (600 queries, each split over several wavefronts, at most 64 output
    positions per wavefront): 172-d f32 rows through memory, LastFM's K = 512 with
    2-d rows, time encodings, queries after and inside their windows."""
    N, b = 400, 200
    rng, g, csr, tmax, fdt = _stream(45 + K, N, d, bf16)
    spec = GatherSpec(neighbors=NeighborSpec(k=K), time_encoding=100, dt_mode=dt_mode)
    pipe = DataPipeline(spec, g)
    assert _shape_m(g, 3 * b, K, 100)[1] > 1  # split: the csr_split shape
    for _ in range(2):
        nodes, qt = _queries(rng, N, 3 * b, tmax)
        src, dst, neg = (np.maximum(nodes[i * b:(i + 1) * b], 0) for i in range(3))
        t = np.where(np.isnan(qt[:b]), tmax + 1.0, qt[:b])
        pb = pipe.prepare(RawBatch(src=cu(src), dst=cu(dst), time=cu(t), neg=cu(neg)))
        allq = np.concatenate([src, dst, neg])
        qts = np.concatenate([t, t, t])
        o = O.recent(allq, qts, K, csr, None, d, fdt)
        assert o.mask.all(1).any() and not o.mask.all()
        groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
        assert np.array_equal(torch.cat([x.neighbor_ids for x in groups]).cpu().numpy(), o.ids)
        assert np.array_equal(torch.cat([x.timestamps for x in groups]).cpu().numpy().view(np.int64),
                              o.times.view(np.int64))
        assert np.array_equal(torch.cat([x.mask for x in groups]).cpu().numpy(), o.mask)
        assert np.array_equal(np.concatenate([_feats_u8(x.edge_feats) for x in groups]),
                              o.feats.view(np.uint8))
        dt = O.dt_dygformer(qts, o.times) if dt_mode == "dygformer" else O.dt_tgn(qts, o.times)
        exp = O.time_encode_exact(dt, cosine_time_weights(100), o.mask if dt_mode == "dygformer" else None)
        got = torch.cat([x.time_enc for x in groups]).cpu().numpy()
        assert np.max(np.abs(got - exp)) <= TE_ATOL


@pytest.mark.parametrize("d,bf16,K,Q", [(3, False, 20, 500), (7, True, 33, 500), (172, False, 64, 3000),
                                        (16, True, 64, 100), (4, False, 300, 3000), (16, True, 512, 700)])
def test_csr_split_recent_matches_oracle(d, bf16, K, Q):
    """recent() launches csr_split takes: 12- and 14-byte rows (4- and 2-byte
    copy chunks), 688-byte rows at 3,000 queries (rows through memory, 4 waves per
    query), a small launch (8 waves per query), K = 300 and 512 (8 waves of at
    most 64 positions); edge ids, NaN query times, padding and out-of-range
    nodes."""
    N = 400
    rng, g, csr, tmax, fdt = _stream(60 + K, N, d, bf16)
    nodes, qt = _queries(rng, N, Q, tmax)
    bad = rng.random(Q) < 0.02
    nodes[bad] = N + 3
    r = g.recent(cu(nodes), cu(qt), K)
    o = O.recent(np.where(bad, -1, nodes), qt, K, csr, None, d, fdt)
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(_feats_u8(r.edge_feats), o.feats.view(np.uint8))
    assert np.array_equal(r.edge_ids.cpu().numpy(), o.eids)
    assert g.status()["bad_query_nodes"] == int(bad.sum())


def _special_graph(seed, N, d, E=6000):
    """A frozen CSR whose times include -0.0 / +0.0 ties, ±inf and NaN (NaN sorts
    after every time, -0.0 ties +0.0 in build order), built from events that are
    not time-ordered (the general build)."""
    rng = np.random.default_rng(seed)
    src = np.minimum(rng.zipf(1.5, E) - 1, N - 1).astype(np.int64)
    dst = rng.integers(0, N, E)
    time = rng.choice(np.array([-0.0, 0.0, -np.inf, np.inf, np.nan, -2.5, 1.0, 3.0, 7.5]), E)
    time = np.where(rng.random(E) < 0.5, np.floor(rng.uniform(-10, 10, E)), time)
    f = rng.standard_normal((E, d)).astype(np.float32)
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=8, track_edge_ids=True)
    events = []
    for lo in range(0, E, 1500):
        hi = min(E, lo + 1500)
        g.advance(cu(src[lo:hi]), cu(dst[lo:hi]), cu(time[lo:hi]), cu(f[lo:hi]))
        events.append((src[lo:hi], dst[lo:hi], time[lo:hi], f[lo:hi], lo))
    g.freeze_csr()
    assert not g._csr_time_sorted  # the general build ran
    return rng, g, O.csr_freeze(N, d, events)


@pytest.mark.parametrize("K,Q", [(20, 3000), (20, 300), (64, 3000), (512, 200)])
def test_ring_less_special_times(K, Q):
    """csr_window (K <= 64, more than 2,048 queries) and csr_split (the rest) on
    windows holding ±0, ±inf and NaN times, queried at ±0, ±inf, NaN and grid times:
    ids, times, rows, masks and edge ids equal to the oracle's."""
    N, d = 60, 4
    rng, g, csr = _special_graph(70 + K, N, d)
    nodes = rng.integers(-1, N, Q)
    qt = rng.choice(np.array([-0.0, 0.0, -np.inf, np.inf, np.nan, 1.0, 3.0, 100.0]), Q)
    qt = np.where(rng.random(Q) < 0.5, np.floor(rng.uniform(-12, 12, Q)), qt)
    r = g.recent(cu(nodes), cu(qt), K)
    o = O.recent(nodes, qt, K, csr, None, d)
    assert o.mask.any() and not o.mask.all()
    assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids)
    assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64))
    assert np.array_equal(r.mask.cpu().numpy(), o.mask)
    assert np.array_equal(r.edge_feats.cpu().numpy(), o.feats)
    assert np.array_equal(r.edge_ids.cpu().numpy(), o.eids)


def test_ring_less_routing_boundaries():
    """Every side of the host's routing of ring-less launches: K = 1, 15, 16, 17, 31,
    32, 33, 63, 64, 65, 128, 129 at 2,048 and 2,049 queries (csr_split with a split,
    csr_window with none) and rows of 16, 48, 64 and 80 bytes (80: csr_split even
    without a split), each against the oracle."""
    N = 300
    for d in (4, 12, 16, 20):
        rng, g, csr, tmax, fdt = _stream(80 + d, N, d, False, E=12000)
        for K in (1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 128, 129):
            for Q in (2048, 2049):
                nodes, qt = _queries(rng, N, Q, tmax)
                r = g.recent(cu(nodes), cu(qt), K)
                o = O.recent(nodes, qt, K, csr, None, d, fdt)
                case = (d, K, Q)
                assert np.array_equal(r.neighbor_ids.cpu().numpy(), o.ids), case
                assert np.array_equal(r.timestamps.cpu().numpy().view(np.int64), o.times.view(np.int64)), case
                assert np.array_equal(r.mask.cpu().numpy(), o.mask), case
                assert np.array_equal(r.edge_feats.cpu().numpy(), o.feats), case
