"""Frozen-CSR build on the device (tgx_csr_build through TemporalGraph.freeze_csr)
against the oracle's csr_freeze (numpy stable argsorts by time, then by node).

Bit-exact offsets, ids, times, feature rows and edge ids over: many equal times
(ties keep build order, -0.0 ties +0.0, NaN sorts last), nodes without
entries, hot nodes, one to several thousand radix tiles (and one build large
enough for a three-level scan of the digit counts), f32 / bf16 / odd / zero
row widths, batches without features, empty builds and out-of-range ids.
"""
import struct

import numpy as np
import pytest
import torch

from oracle import spec as O
from tgengine_amd import TemporalGraph
from tgengine_amd.core import _lib
from tgengine_amd.synthetic import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _build(N, d, bf16, batches, eids=False):
    """Pre-freeze advance() of every batch on the device graph, then freeze; the
    oracle gets the same events."""
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda",
                      feat_dtype=torch.bfloat16 if bf16 else torch.float32, track_edge_ids=eids)
    events, eb = [], 0
    for (src, dst, time, feat) in batches:
        b = len(src)
        f_dev = None
        if feat is not None:
            t = torch.from_numpy(np.ascontiguousarray(feat))
            f_dev = (t.view(torch.bfloat16) if bf16 else t).cuda()
        g.advance(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda(),
                  torch.from_numpy(time).cuda(), f_dev)
        fo = feat if feat is not None else np.zeros((b, d), np.uint16 if bf16 else np.float32)
        events.append((src, dst, time, fo, eb))
        eb += b
    g.freeze_csr()
    ref = O.csr_freeze(N, d, events, np.uint16 if bf16 else np.float32)
    return g, ref


def _compare(g, ref, where=""):
    assert np.array_equal(g._offsets.cpu().numpy(), ref.offsets), f"{where} offsets"
    assert np.array_equal(g._nbr_ids.cpu().numpy(), ref.ids), f"{where} ids"
    assert np.array_equal(g._nbr_times.cpu().numpy().view(np.int64),
                          ref.times.view(np.int64)), f"{where} times"
    f = g._nbr_feats
    f = f.view(torch.int16).cpu().numpy().view(np.uint16) if f.dtype == torch.bfloat16 else f.cpu().numpy()
    assert np.array_equal(f.view(np.uint8), np.ascontiguousarray(ref.feats).view(np.uint8)), f"{where} feats"
    if g._nbr_eids is not None:
        assert np.array_equal(g._nbr_eids.cpu().numpy(), ref.eids), f"{where} eids"
    st = g.status()
    assert st["bad_event_nodes"] == 0, st


def _feat(rng, b, d, bf16):
    f = rng.standard_normal((b, d)).astype(np.float32)
    return f32_to_bf16_bits(f) if bf16 else f


def _batches(rng, N, sizes, d, bf16, tie_grid=None, feat_every=1, node_hi=None):
    out = []
    hi = node_hi or N
    for k, b in enumerate(sizes):
        src = rng.integers(0, hi, b)
        dst = rng.integers(0, hi, b)
        src[: b // 5] = 3 % N  # a hot node
        t = rng.uniform(-50, 1000, b)
        if tie_grid:
            t = np.round(t / tie_grid) * tie_grid  # many equal times
        feat = _feat(rng, b, d, bf16) if (feat_every and k % feat_every == 0) else None
        out.append((src.astype(np.int64), dst.astype(np.int64), t.astype(np.float64), feat))
    return out


@pytest.mark.parametrize("d,bf16,eids", [(16, True, False), (172, False, True), (5, True, True),
                                         (0, False, False), (3, False, False)])
def test_csr_build_matches_the_oracle(d, bf16, eids):
    rng = np.random.default_rng(10 + d)
    N = 5000
    batches = _batches(rng, N, [700, 1, 3000, 0, 2500], d, bf16, tie_grid=5.0, feat_every=2,
                       node_hi=N - 700)  # the top 700 nodes stay empty
    g, ref = _build(N, d, bf16, batches, eids)
    _compare(g, ref)


def test_csr_build_signed_zero_and_nan_times():
    rng = np.random.default_rng(11)
    N, b = 50, 400
    src = rng.integers(0, N, b).astype(np.int64)
    dst = rng.integers(0, N, b).astype(np.int64)
    t = rng.choice(np.array([-0.0, 0.0, -1.5, 2.0, np.nan, -np.inf, np.inf, 1e-300, -1e-300]), b)
    g, ref = _build(N, 4, False, [(src, dst, t.astype(np.float64), _feat(rng, b, 4, False))], True)
    _compare(g, ref)


def test_csr_build_single_node_and_single_entry():
    g, ref = _build(1, 2, False, [(np.zeros(3, np.int64), np.zeros(3, np.int64),
                                   np.array([3.0, 1.0, 2.0]), np.ones((3, 2), np.float32))])
    _compare(g, ref)
    g, ref = _build(7, 2, True, [(np.array([6], np.int64), np.array([0], np.int64),
                                  np.array([5.0]), None)])
    _compare(g, ref)


def test_csr_build_empty():
    g, ref = _build(10, 4, False, [])
    _compare(g, ref)
    g, ref = _build(10, 4, False, [(np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(0), None)])
    _compare(g, ref)


def test_csr_build_many_tiles_and_wide_node_ids():
    # 2.4M entries (1,200 radix tiles), node ids over 21 bits (three node passes)
    rng = np.random.default_rng(12)
    N = 1_500_000
    batches = _batches(rng, N, [400_000, 800_000], 4, True, tie_grid=0.25)
    g, ref = _build(N, 4, True, batches, True)
    _compare(g, ref)


def test_csr_build_three_level_count_scan():
    # 34M entries: 16,602 tiles x 256 digits = 4.25M counts > 2048^2, so the
    # exclusive scan of the digit counts recurses twice
    rng = np.random.default_rng(13)
    N, b = 100_000, 17_000_000
    src = rng.integers(0, N, b).astype(np.int64)
    dst = rng.integers(0, N, b).astype(np.int64)
    t = np.round(rng.uniform(0, 1e6, b)).astype(np.float64)
    g, ref = _build(N, 0, False, [(src, dst, t, None)], True)
    _compare(g, ref)


def _ordered_batches(rng, N, sizes, d, bf16, feat_every=2, node_hi=None):
    """A time-ordered stream: times strictly increasing within every batch, each
    batch starting at its predecessor's last time (a tie across the boundary)."""
    out, t = [], 100.0
    hi = node_hi or N
    for k, b in enumerate(sizes):
        tt = t + np.cumsum(rng.exponential(1.0, b) + 1e-3)
        if k > 0 and b > 0:
            tt[0] = t
        if b > 0:
            t = float(tt[-1])
        src = rng.integers(0, hi, b)
        src[: b // 5] = 3 % N  # a hot node
        feat = _feat(rng, b, d, bf16) if (feat_every and k % feat_every == 0) else None
        out.append((src.astype(np.int64), rng.integers(0, hi, b).astype(np.int64), tt.astype(np.float64), feat))
    return out


@pytest.mark.parametrize("d,bf16,eids,N", [(16, True, True, 5000), (172, False, False, 300),
                                           (3, False, True, 200_000), (0, False, False, 70_000)])
def test_csr_build_time_ordered_stream(d, bf16, eids, N):
    """A time-ordered stream is built from its events in pairs (node passes only):
    the same CSR as the oracle's two stable sorts of the build order."""
    rng = np.random.default_rng(20 + d)
    batches = _ordered_batches(rng, N, [500, 1, 0, 2000, 777, 3], d, bf16, node_hi=N - 50)
    g, ref = _build(N, d, bf16, batches, eids)
    assert g._csr_time_sorted
    _compare(g, ref)


@pytest.mark.parametrize("where", ["tie", "step_back", "nan"])
def test_csr_build_almost_ordered_stream_sorts_by_time(where):
    """One tie inside a batch, one step back in time, or a NaN: the stream is not
    time-ordered.  With the tie it still never decreases, and the build takes the
    time order from runs of equal times; otherwise it sorts the build order (formed
    on the device from the events and the calls' first events) by time first."""
    rng = np.random.default_rng(30)
    batches = _ordered_batches(rng, 40, [300, 300, 300], 4, False)
    t = batches[1][2]
    if where == "tie":
        t[100] = t[99]
    elif where == "step_back":
        t[150] = t[10] - 1.0
    else:
        t[7] = np.nan
    g, ref = _build(40, 4, False, batches, True)
    assert not g._csr_time_sorted
    assert g._csr_build_mode == ("runs" if where == "tie" else "sort")
    _compare(g, ref)


def _tied_batches(rng, N, sizes, d, bf16, grid, node_hi=None):
    """A non-decreasing stream with many equal times: a running clock rounded down
    to multiples of grid, so runs of equal times span events inside a batch and
    reach across batch boundaries (each batch starts at its predecessor's last
    time or later)."""
    out, t = [], 10.0
    hi = node_hi or N
    for k, b in enumerate(sizes):
        tt = np.floor((t + np.cumsum(rng.exponential(grid / 3, b))) / grid) * grid
        if b > 0:
            if k % 2 == 1:
                tt[0] = t  # the previous batch's last time
            tt = np.maximum.accumulate(np.maximum(tt, t))
            t = float(tt[-1])
        src = rng.integers(0, hi, b)
        src[: b // 5] = 3 % N  # a hot node
        feat = _feat(rng, b, d, bf16) if k % 2 == 0 else None
        out.append((src.astype(np.int64), rng.integers(0, hi, b).astype(np.int64), tt.astype(np.float64), feat))
    return out


@pytest.mark.parametrize("d,bf16,eids,N,sizes,grid", [
    (16, True, True, 5000, [500, 1, 0, 2000, 777, 3, 1, 1], 1.0),
    (172, False, False, 300, [300, 300, 300], 10.0),
    (0, False, True, 70_000, [1, 1, 1, 5, 4000], 1e6),
    (4, True, False, 1_000_000, [2_500_000, 2_500_000], 0.5),
])
def test_csr_build_nondecreasing_stream_uses_runs(d, bf16, eids, N, sizes, grid):
    """Ties everywhere but time never going down: the build order's stable time
    order comes from runs of equal times within each call (no time passes); the
    same CSR as the oracle's two stable sorts.  The last case has 5M events, so
    the scan of the run marks has two levels."""
    rng = np.random.default_rng(40 + d)
    batches = _tied_batches(rng, N, sizes, d, bf16, grid, node_hi=N - 50)
    g, ref = _build(N, d, bf16, batches, eids)
    assert g._csr_build_mode == "runs"
    _compare(g, ref)


def test_csr_build_runs_with_signed_zero_and_infinity():
    """-0.0 ties +0.0 and +inf ties +inf in a non-decreasing stream."""
    rng = np.random.default_rng(44)
    t1 = np.array([-5.0, -0.0, 0.0, -0.0, 0.0, 1.0, 1.0])
    t2 = np.array([1.0, 1.0, 2.0, np.inf, np.inf])
    batches = [(rng.integers(0, 9, len(t)).astype(np.int64), rng.integers(0, 9, len(t)).astype(np.int64), t,
                _feat(rng, len(t), 4, False)) for t in (t1, t2)]
    g, ref = _build(9, 4, False, batches, True)
    assert g._csr_build_mode == "runs"
    _compare(g, ref)


def _scan(src, dst, t, starts):
    """tgx_csr_scan on device copies: (lo, hi, order level, largest non-NaN time);
    the level is 2 for a time-ordered stream, 1 for a non-decreasing one, else 0."""
    L = _lib.lib()
    s, d, tt = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (src, dst, t))
    st = torch.tensor(starts, dtype=torch.int64, device="cuda")
    ws = torch.empty(int(L.tgx_csr_scan_workspace_size()), dtype=torch.uint8, device="cuda")
    out = torch.full((4,), 7, dtype=torch.int64, device="cuda")
    assert L.tgx_csr_scan(s.data_ptr(), d.data_ptr(), tt.data_ptr(), len(src), st.data_ptr() if len(starts) else None,
                          len(starts), out.data_ptr(), ws.data_ptr(), ws.numel(), None) == 0
    lo, hi, ordered, bits = out.cpu().tolist()
    return lo, hi, ordered, struct.unpack("<d", struct.pack("<q", bits))[0]


@pytest.mark.parametrize("E", [1, 2, 255, 1024, 1025, 262_145, 1_500_001])
def test_csr_scan_known_cases(E):
    """The pre-freeze scan on streams whose answers are fixed by construction:
    strictly increasing times with ties only at call starts are ordered; one tie
    inside a call, a step back, a NaN or inf followed by inf is not, wherever it
    sits (first step, a workgroup boundary, the last event); the node range comes
    from planted extremes and the largest time skips NaN."""
    rng = np.random.default_rng(E)
    t = np.cumsum(rng.uniform(0.5, 1.5, E))
    starts = sorted({0, *rng.integers(1, E, min(E - 1, 50)).tolist()}) if E > 1 else [0]
    for k in starts[1:]:  # tie each call's first event with the previous one
        t[k:] -= t[k] - t[k - 1]
        t[k] = t[k - 1]
    src = rng.integers(10, 1000, E)
    dst = rng.integers(10, 1000, E)
    src[-1], dst[E // 2] = 3, 5000
    lo, hi, ordered, tmax = _scan(src, dst, t, starts)
    assert (lo, hi, ordered, tmax) == (min(3, int(dst.min())), 5000, 2, float(t.max()))
    if E < 2:
        return
    inner = [k for k in (1, E // 2, 1024, 4 * 256 * 1024, E - 1) if 0 < k < E and k not in starts]
    for k in inner:
        for kind in ("tie", "back", "nan", "inf"):
            u = t.copy()
            if kind == "tie":
                u[k] = u[k - 1]
            elif kind == "back":
                u[k] = u[k - 1] - 1e-9
            elif kind == "nan":
                u[k] = np.nan
            else:
                u[k - 1] = u[k] = np.inf
            got = _scan(src, dst, u, starts)
            # a tie inside a call, or inf, inf at the very end, still never decreases
            nondecreasing = kind == "tie" or (kind == "inf" and k == E - 1)
            assert got[2] == (1 if nondecreasing else 0), (k, kind)
            want = np.inf if kind == "inf" else float(np.nanmax(u))
            assert got[3] == want, (k, kind)
    # -0.0 after +0.0 is a zero step: time-ordered only at a call start, and
    # non-decreasing either way
    z = np.zeros(2)
    z[1] = -0.0
    assert _scan(src[:2], dst[:2], z, [0, 1])[2] == 2
    assert _scan(src[:2], dst[:2], z, [0])[2] == 1
    assert _scan(src[:2], dst[:2], z, [0, 1, 1])[2] == 2  # a repeated start counts once
    # times 0, 0, 1, 1, 2, 2, ...: zero steps at every odd event break the strict
    # order unless every odd event starts a call; the stream never decreases
    u = np.repeat(np.arange(E // 2 + 1, dtype=np.float64), 2)[:E]
    assert _scan(src, dst, u, list(range(0, E, 2)))[2] == 1
    assert _scan(src, dst, u, list(range(1, E, 2)))[2] == 2
    # every time NaN: no largest time
    assert _scan(src[:2], dst[:2], np.full(2, np.nan), [0, 1])[3] == -np.inf


def test_csr_build_rejects_out_of_range_nodes():
    g = TemporalGraph(10, edge_feat_dim=2, device="cuda")
    g.advance(torch.tensor([1, 10], device="cuda"), torch.tensor([2, 3], device="cuda"),
              torch.tensor([1.0, 2.0], device="cuda", dtype=torch.float64))
    with pytest.raises(IndexError):
        g.freeze_csr()


def test_prefreeze_values_are_copied_at_advance_time():
    """Changing the caller's tensors after advance() does not change the CSR (the
    reference copies them into host lists)."""
    rng = np.random.default_rng(14)
    N, b, d = 100, 64, 4
    src = torch.from_numpy(rng.integers(0, N, b)).cuda()
    dst = torch.from_numpy(rng.integers(0, N, b)).cuda()
    t = torch.from_numpy(rng.uniform(0, 10, b)).cuda()
    f = torch.from_numpy(_feat(rng, b, d, False)).cuda()
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda")
    g.advance(src, dst, t, f)
    ref = O.csr_freeze(N, d, [(src.cpu().numpy(), dst.cpu().numpy(), t.cpu().numpy(), f.cpu().numpy(), 0)])
    src.fill_(0)
    t.fill_(0.0)
    f.fill_(7.0)
    g.freeze_csr()
    _compare(g, ref)
