"""Ring update (tgx_ring_append through TemporalGraph.advance) against the oracle.

Bit-exact comparison of ids, times, feature rows, write positions and edge ids
after every batch, over shapes that reach every code path of both update
designs: the two-launch path (batches of up to 32768 entries: the plan ranks
every entry among its node's entries in entry order from an LDS hash of its
workgroup's nodes and one scan of the batch, in 1,024-thread workgroups, or
256 for batches of at most 256 entries; the commit is one copy per entry) and
the four-launch path (larger batches: tickets from node-indexed counters, small
groups of 2..64 entries, large groups over one or several bitmap windows), plus
B not a power of two, bf16 rows of odd width, zero-width rows, invalid node ids,
the size boundary between the two paths, plan-workgroup boundaries, and batch
shapes that give every node the same number of entries (one node holding the
batch, consecutive ids in pairs or groups).
"""
import numpy as np
import pytest
import torch

from oracle import spec as O
from tgengine_amd import TemporalGraph

pytestmark = pytest.mark.gpu


def _feat(rng, b, d, bf16):
    f = rng.standard_normal((b, d)).astype(np.float32)
    if bf16:
        from tgengine_amd.synthetic import f32_to_bf16_bits
        return f32_to_bf16_bits(f)
    return f


def _to_dev(f, bf16):
    t = torch.from_numpy(np.ascontiguousarray(f))
    return (t.view(torch.bfloat16) if bf16 else t).cuda()


def _graph_and_ring(N, B, d, bf16, eids=False):
    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=B,
                      feat_dtype=torch.bfloat16 if bf16 else torch.float32, track_edge_ids=eids)
    g.freeze_csr()  # empty CSR: every advance goes to the ring
    ring = O.Ring.empty(N, B, d, np.uint16 if bf16 else np.float32, with_eids=eids)
    return g, ring


def _compare(g, ring, where):
    assert np.array_equal(g._ov_ids.cpu().numpy(), ring.ids), f"{where}: ids"
    assert np.array_equal(g._ov_times.cpu().numpy().view(np.int64), ring.times.view(np.int64)), f"{where}: times"
    gf = g._ov_feats
    gf = gf.view(torch.int16).cpu().numpy().view(np.uint16) if gf.dtype == torch.bfloat16 else gf.cpu().numpy()
    assert np.array_equal(gf.view(np.uint8), ring.feats.view(np.uint8)), f"{where}: feats"
    assert np.array_equal(g._ov_write_pos.cpu().numpy(), ring.wp), f"{where}: write_pos"
    if ring.eids is not None:
        assert np.array_equal(g._ov_eids.cpu().numpy(), ring.eids), f"{where}: eids"
    N = g.num_nodes
    assert int(g._ov_scratch[:N].abs().sum()) == 0, f"{where}: node counters not restored to zero"


def _run(seed, N, B, d, bf16, batches, eids=False):
    rng = np.random.default_rng(seed)
    g, ring = _graph_and_ring(N, B, d, bf16, eids)
    eb = 0
    for bi, (src, dst) in enumerate(batches(rng)):
        b = len(src)
        t0 = 10.0 * (2 * b + 10) * (bi + 1)
        time = t0 + np.cumsum(rng.exponential(1.0, b) + 1e-3)
        f = _feat(rng, b, d, bf16)
        g.advance(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda(),
                  torch.from_numpy(time).cuda(), _to_dev(f, bf16))
        O.ring_advance(ring, src, dst, time, f, eid_base=eb)
        eb += b
        _compare(g, ring, f"seed {seed} batch {bi}")
    st = g.status()
    assert st == {"bad_event_nodes": 0, "key_collisions": 0, "bad_query_nodes": 0}, st


def _uniform(N, b, nb):
    def gen(rng):
        for _ in range(nb):
            yield rng.integers(0, N, b), rng.integers(0, N, b)
    return gen


def _hot(N, b, nb, hot_frac):
    def gen(rng):
        for _ in range(nb):
            src = rng.integers(0, N, b)
            dst = rng.integers(0, N, b)
            m = rng.random(b) < hot_frac
            src = np.where(m, 7 % N, src)
            m2 = rng.random(b) < hot_frac / 2
            dst = np.where(m2, 7 % N, dst)
            yield src, dst
    return gen


@pytest.mark.parametrize("B", [1, 2, 7, 32, 64])
def test_ring_small_nodes_many_groups(B):
    _run(1, 50, B, 16, False, _uniform(50, 300, 6))


# rows past 1 KB (300 f32, 2048 bf16) take more than one round of a group's copy
@pytest.mark.parametrize("d,bf16", [(0, False), (1, False), (3, True), (5, True), (16, True),
                                    (172, False), (512, True), (37, False), (300, False),
                                    (2048, True)])
def test_ring_row_widths(d, bf16):
    _run(2, 200, 8, d, bf16, _hot(200, 500, 4, 0.2))


def test_ring_large_group_single_window():
    # node 7 takes ~45% of 4000 events as src -> ~1800 + entries in one batch
    _run(3, 100_000, 32, 16, True, _hot(100_000, 4000, 3, 0.45))


def test_ring_large_group_many_windows():
    """A node with > 64 entries whose last B are spread over more than one
    8192-index window (batch of 20000 events = 40000 entries)."""
    def gen(rng):
        for _ in range(2):
            b = 20000
            src = rng.integers(100, 5000, b)
            dst = rng.integers(100, 5000, b)
            src[::300] = 3           # 67 entries, 300 events apart
            dst[-5::-97] = 4         # ~206 dst-role entries of node 4
            yield src, dst
    _run(4, 5000, 64, 4, False, gen)


def test_ring_self_loops_and_edge_ids():
    def gen(rng):
        for _ in range(5):
            src = rng.integers(0, 30, 120)
            dst = np.where(rng.random(120) < 0.3, src, rng.integers(0, 30, 120))
            yield src, dst
    _run(5, 30, 16, 8, False, gen, eids=True)


def test_ring_batch_larger_than_16384_entries():
    _run(6, 300_000, 32, 8, True, _hot(300_000, 12000, 2, 0.05))


def _windows_gen(b, nb):
    """Nodes 3 and 4 with > 64 entries spread over several 8192-index windows,
    the rest groups of a few entries each."""
    def gen(rng):
        for _ in range(nb):
            src = rng.integers(100, 5000, b)
            dst = rng.integers(100, 5000, b)
            src[:: b // 60] = 3
            dst[-5::-97] = 4
            yield src, dst
    return gen


def test_ring_two_launch_large_group_many_windows():
    # 16000 events = 32000 entries: the two-launch path, four bitmap windows
    _run(8, 5000, 64, 4, False, _windows_gen(16000, 2))


@pytest.mark.parametrize("b", [16384, 16385])
def test_ring_two_and_four_launch_size_boundary(b):
    # 32768 entries (last two-launch size) and 32770 (first four-launch size)
    _run(9, 20_000, 32, 8, True, _windows_gen(b, 2))


def test_ring_odd_batch_masks_stale_entry_nodes():
    """n = 2b with b odd: the commit reads the plan's entry-node array in 16-byte
    groups from the top, so its first read covers two entries past the batch,
    left there by the previous, larger batch.  Node 7 sits at exactly those two
    positions (entries 1998 and 1999 of a 1001-event batch) and is a large group
    of the next 999-event batches: with fewer entries than B (every entry kept)
    and with more (only the top B)."""
    def gen(rng):
        src = rng.integers(100, 5000, 1001)
        dst = rng.integers(100, 5000, 1001)
        dst[997:999] = 7  # entries 1001 + 997 and 1001 + 998
        src[::50] = 7
        yield src, dst
        for step in (40, 9):  # 25 entries of node 7 (< B), then 111 (> B)
            src = rng.integers(100, 5000, 999)
            dst = rng.integers(100, 5000, 999)
            src[::step] = 7
            yield src, dst
            src = rng.integers(100, 5000, 1001)  # refill the stale positions
            dst = rng.integers(100, 5000, 1001)
            dst[997:999] = 7
            yield src, dst
    _run(11, 5000, 32, 8, False, gen)


def test_ring_list_capacity_edges():
    """Groups of exactly 7, 8, 9 and 10 entries (a full node list, and the first
    overflow entries) next to singletons, for B below and above the group size."""
    def gen(rng):
        for _ in range(4):
            nodes = np.concatenate([np.repeat(np.arange(4), [7, 8, 9, 10]),
                                    rng.integers(10, 1000, 266)])
            rng.shuffle(nodes)
            src = nodes[:150]
            dst = nodes[150:]
            yield src, dst
    for B in (4, 8, 9, 16):
        _run(10, 1000, B, 8, False, gen)


def test_ring_invalid_ids_are_skipped_and_flagged():
    rng = np.random.default_rng(7)
    N, B, d = 20, 4, 2
    g, ring = _graph_and_ring(N, B, d, False)
    src = np.array([1, 2, 25, -3, 4], np.int64)
    dst = np.array([2, 30, 3, 4, 1], np.int64)
    time = 100.0 + np.arange(5, dtype=np.float64)
    f = rng.standard_normal((5, d)).astype(np.float32)
    g.advance(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda(),
              torch.from_numpy(time).cuda(), torch.from_numpy(f).cuda())
    # oracle: drop the directed entries whose `from` is out of range
    keep_s = (src >= 0) & (src < N)
    keep_d = (dst >= 0) & (dst < N)
    frm = np.concatenate([src, dst]); ok = np.concatenate([keep_s, keep_d])
    assert int(g.status()["bad_event_nodes"]) == int((~ok).sum()) == 3
    # entries from valid nodes land exactly as the rule says (checked by brute force)
    for u in range(N):
        ent = [i for i in range(10) if ok[i] and frm[i] == u]
        got = g._ov_ids[u].cpu().numpy()
        assert (got != -1).sum() == min(len(ent), B)
    assert int(g._ov_scratch[:N].abs().sum()) == 0


def test_ring_key_collision_is_flagged():
    g, _ = _graph_and_ring(10, 4, 2, False)
    b = 100
    time = np.arange(b, dtype=np.float64) * 0.01  # int(max t)+2 = 2 <= 2b-1
    g.advance(torch.arange(b).remainder(10).cuda(), torch.arange(b).remainder(7).cuda(),
              torch.from_numpy(time).cuda(), torch.zeros(b, 2).cuda())
    assert g.status()["key_collisions"] == 1


def test_ring_empty_batch_is_a_noop():
    g, ring = _graph_and_ring(10, 4, 2, False)
    g.advance(torch.empty(0, dtype=torch.int64).cuda(), torch.empty(0, dtype=torch.int64).cuda(),
              torch.empty(0, dtype=torch.float64).cuda(), torch.empty(0, 2).cuda())
    _compare(g, ring, "empty")
    assert g.num_edges == 0


def test_ring_zero_features_when_edge_feat_is_none():
    rng = np.random.default_rng(8)
    g, ring = _graph_and_ring(40, 8, 6, False)
    src = rng.integers(0, 40, 64)
    dst = rng.integers(0, 40, 64)
    time = 500.0 + np.arange(64, dtype=np.float64)
    g.advance(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda(), torch.from_numpy(time).cuda())
    O.ring_advance(ring, src, dst, time, np.zeros((64, 6), np.float32))
    _compare(g, ring, "no feats")


# ------------------------------------------------------------- planned updates
# TemporalGraph.plan_append enqueues the first half of a batch's ring update
# (DataPipeline.prepare runs the same plan inside its gather launch); advance()
# commits the plan when it receives the same src/dst/time tensors, otherwise
# discards it.  Every path must leave the ring exactly as the oracle's update,
# with the node counters back at zero.

def _stream_batches(rng, N, n_batches, b, hot=3):
    out = []
    for bi in range(n_batches):
        src = rng.integers(0, N, b)
        dst = rng.integers(0, N, b)
        src[: b // 4] = rng.integers(0, hot, b // 4)  # repeated nodes -> small/large groups
        t0 = 10.0 * (2 * b + 10) * (bi + 1)
        time = t0 + np.cumsum(rng.exponential(1.0, b) + 1e-3)
        out.append((src.astype(np.int64), dst.astype(np.int64), time))
    return out


def _dev(src, dst, time, feat, bf16):
    return (torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda(), torch.from_numpy(time).cuda(),
            _to_dev(feat, bf16))


@pytest.mark.parametrize("bf16", [False, True])
def test_planned_updates_match_the_oracle(bf16):
    rng = np.random.default_rng(41)
    N, B, d = 300, 8, 8 if bf16 else 6
    g, ring = _graph_and_ring(N, B, d, bf16)
    for bi, (src, dst, time) in enumerate(_stream_batches(rng, N, 6, 700)):
        feat = _feat(rng, len(src), d, bf16)
        s, t_dst, t, f = _dev(src, dst, time, feat, bf16)
        assert g.plan_append(s, t_dst, t) == (bi > 0)  # the ring exists from the first advance on
        g.advance(s, t_dst, t, f)
        O.ring_advance(ring, src, dst, time, feat)
        _compare(g, ring, f"planned batch {bi}")
    assert all(v == 0 for v in g.status().values())


@pytest.mark.parametrize("b,nb", [(300, 5), (17000, 2)])  # two- and four-launch paths
def test_plan_discarded_when_advance_gets_other_tensors(b, nb):
    rng = np.random.default_rng(42)
    N, B, d = 200, 4, 4
    g, ring = _graph_and_ring(N, B, d, False)
    batches = _stream_batches(rng, N, nb, b)
    for bi, (src, dst, time) in enumerate(batches):
        feat = _feat(rng, len(src), d, False)
        s, t_dst, t, f = _dev(src, dst, time, feat, False)
        g.plan_append(s, t_dst, t)
        if bi % 2:
            # equal values in other tensors: the plan is dropped, the batch still applies
            g.advance(s.clone(), t_dst.clone(), t.clone(), f)
        else:
            # a plan for a batch that never comes, then the real one
            other = _stream_batches(rng, N, 1, b)[0]
            o = _dev(*other, _feat(rng, b, d, False), False)
            g.plan_append(o[0], o[1], o[2])
            g.advance(s, t_dst, t, f)
        O.ring_advance(ring, src, dst, time, feat)
        _compare(g, ring, f"batch {bi}")
    assert all(v == 0 for v in g.status().values())


def test_plan_sees_in_place_changes_and_reports_status_once():
    rng = np.random.default_rng(43)
    N, B, d = 100, 4, 2
    g, ring = _graph_and_ring(N, B, d, False)
    (src, dst, time), (src2, dst2, time2) = _stream_batches(rng, N, 2, 200)
    feat = _feat(rng, 200, d, False)
    s, t_dst, t, f = _dev(src, dst, time, feat, False)
    g.advance(s, t_dst, t, f)  # allocates the ring
    O.ring_advance(ring, src, dst, time, feat)
    # plan a batch, then change it in place: the version counter forces a re-plan
    feat2 = _feat(rng, 200, d, False)
    s2, d2, t2, f2 = _dev(src2, dst2, time2, feat2, False)
    g.plan_append(s2, d2, t2)
    src2 = src2.copy()
    src2[:10] = np.arange(10)
    s2[:10] = torch.arange(10, device="cuda")
    g.advance(s2, d2, t2, f2)
    O.ring_advance(ring, src2, dst2, time2, feat2)
    _compare(g, ring, "after in-place change")
    # out-of-range node ids in a planned batch are reported once, at the commit
    (src3, dst3, time3), = _stream_batches(rng, N, 1, 200)
    src3 = src3.copy()
    src3[:3] = N + 5
    feat3 = _feat(rng, 200, d, False)
    s3, d3, t3, f3 = _dev(src3, dst3, time3, feat3, False)
    g.plan_append(s3, d3, t3)
    g.advance(s3, d3, t3, f3)
    assert g.status()["bad_event_nodes"] == 3
    N_ = g.num_nodes
    assert int(g._ov_scratch[:N_].abs().sum()) == 0


def test_restore_and_reset_drop_a_pending_plan():
    rng = np.random.default_rng(44)
    N, B, d = 80, 4, 2
    g, ring = _graph_and_ring(N, B, d, False)
    (a, b_, c), (a2, b2, c2) = _stream_batches(rng, N, 2, 100)
    feat = _feat(rng, 100, d, False)
    s, t_dst, t, f = _dev(a, b_, c, feat, False)
    g.advance(s, t_dst, t, f)
    O.ring_advance(ring, a, b_, c, feat)
    snap = g.snapshot()
    s2, d2, t2, f2 = _dev(a2, b2, c2, _feat(rng, 100, d, False), False)
    g.plan_append(s2, d2, t2)
    g.restore(snap)
    assert g._plan is None
    _compare(g, ring, "restored with a plan pending")
    g.plan_append(s2, d2, t2)
    g.reset()
    assert g._plan is None


@pytest.mark.parametrize("b", [1, 2, 127, 128, 129, 511, 512, 513, 1537, 4096])
def test_ring_plan_workgroup_boundaries(b):
    """Entries of one node on both sides of plan-workgroup boundaries (256-entry
    workgroups up to 256 entries, 1,024 above), a hub in every workgroup, and
    wavefronts holding a node more than once."""
    def gen(rng):
        for _ in range(3):
            src = rng.integers(0, 40, b)
            dst = rng.integers(0, 40, b)
            src[::3] = 5
            yield src, dst
    _run(20 + b, 40, 32, 8, True, gen)


def _shape(name, b):
    """src, dst of a batch whose nodes all have the same number of entries, on
    consecutive ids from a moving base (the multiplicative hash spreads such runs
    evenly, the case a probe scheme must not degrade on)."""
    i = np.arange(b, dtype=np.int64)
    groups = {"pairs": b, "groups8": b // 4, "groups10": b // 5, "groups100": b // 50}

    def gen(rng):
        for j in range(3):
            base = 1000 + 9973 * j
            if name == "singletons":
                yield base + 2 * i, base + 2 * i + 1
            elif name == "one_node":
                yield np.full(b, base), np.full(b, base)
            else:
                g = groups[name]
                yield base + i % g, base + (i + 7) % g
    return gen


@pytest.mark.parametrize("shape", ["singletons", "one_node", "pairs", "groups8", "groups10", "groups100"])
def test_ring_update_shapes_match_the_oracle(shape):
    _run(30, 50_000, 32, 16, True, _shape(shape, 4000))

