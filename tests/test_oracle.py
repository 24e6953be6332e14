"""Pins the CPU oracle (oracle/spec.py) before it is trusted as the parity checker.

Every oracle function is checked against at least one of: a known answer restated
from the reference's own tests, a brute-force twin written independently, or a
closed form.  ``test_planted_*`` plant plausible mistakes into copies of the
oracle and show that the checks catch them.
"""
import numpy as np
import pytest

from oracle import spec as O


def _rand_batches(rng, N, nb, b, d, hot=None, t0=None):
    out = []
    t = float(2 * b + 100) if t0 is None else t0
    for _ in range(nb):
        src = rng.integers(0, N, b)
        dst = rng.integers(0, N, b)
        if hot is not None:
            m = rng.random(b) < 0.5
            src = np.where(m, hot, src)
        gaps = rng.exponential(1.0, b) + 1e-3
        time = t + np.cumsum(gaps)
        t = float(time[-1])
        feat = rng.standard_normal((b, d)).astype(np.float32)
        out.append((src.astype(np.int64), dst.astype(np.int64), time, feat))
    return out


# ---------------------------------------------------------------- ring update
@pytest.mark.parametrize("seed,N,B,b,hot", [(0, 7, 4, 13, None), (1, 30, 8, 40, 3), (2, 5, 2, 9, 0),
                                             (3, 200, 32, 100, 17), (4, 3, 64, 150, 1)])
def test_ring_advance_matches_bruteforce(seed, N, B, b, hot):
    rng = np.random.default_rng(seed)
    d = 3
    r1 = O.Ring.empty(N, B, d, with_eids=True)
    r2 = O.Ring.empty(N, B, d, with_eids=True)
    eb = 0
    for (s, t_, tm, f) in _rand_batches(rng, N, 6, b, d, hot):
        O.ring_advance(r1, s, t_, tm, f, eid_base=eb)
        O.ring_advance_brute(r2, s, t_, tm, f, eid_base=eb)
        eb += len(s)
        assert np.array_equal(r1.ids, r2.ids)
        assert np.array_equal(r1.times, r2.times)
        assert np.array_equal(r1.feats, r2.feats)
        assert np.array_equal(r1.wp, r2.wp)
        assert np.array_equal(r1.eids, r2.eids)


def test_ring_advance_write_pos_closed_form():
    """write_pos grows by min(c, B) per node per batch (temporal_graph.py:365-387)."""
    rng = np.random.default_rng(7)
    N, B, d = 11, 4, 2
    r = O.Ring.empty(N, B, d)
    exp = np.zeros(N, np.int64)
    for (s, t_, tm, f) in _rand_batches(rng, N, 5, 30, d, hot=2):
        c = np.bincount(np.concatenate([s, t_]), minlength=N)
        exp += np.minimum(c, B)
        O.ring_advance(r, s, t_, tm, f)
        assert np.array_equal(r.wp, exp)


def test_ring_keeps_concat_order_not_time():
    """A node with more than B entries in one batch keeps the last B in
    [src-role ..., dst-role ...] order, not the B most recent (temporal_graph.py:125-128, :357-373)."""
    B = 2
    r = O.Ring.empty(5, B, 1)
    # node 0 is src at t=1,2 and dst at t=0.5 (event 2) -> concat order src(1), src(2), dst(0.5)
    src = np.array([0, 0, 3], np.int64)
    dst = np.array([1, 2, 0], np.int64)
    time = np.array([1.0, 2.0, 0.5]) + 10.0
    feat = np.zeros((3, 1), np.float32)
    O.ring_advance(r, src, dst, time, feat)
    # kept for node 0: last 2 of [to=1 @11, to=2 @12, to=3 @10.5] -> (2 @12, 3 @10.5) in slots 0, 1
    assert r.ids[0].tolist() == [2, 3]
    assert r.times[0].tolist() == [12.0, 10.5]
    assert r.wp[0] == 2
    # second batch, node 0 gets one entry -> slot (2 + 0) % 2 = 0
    O.ring_advance(r, np.array([0]), np.array([4]), np.array([20.0]), np.zeros((1, 1), np.float32))
    assert r.ids[0].tolist() == [4, 3] and r.wp[0] == 3


def test_ring_slot_rule_overflowing_batch():
    """c > B in one batch: slots (wp + m) % B for the kept entries, wp += B."""
    B = 3
    r = O.Ring.empty(2, B, 1)
    r.wp[0] = 5
    src = np.zeros(5, np.int64)
    dst = np.ones(5, np.int64)
    time = np.arange(5, dtype=np.float64) + 20.0
    O.ring_advance(r, src, dst, time, np.zeros((5, 1), np.float32))
    # node 0 entries (src role) times 20..24, keep 22, 23, 24 at slots 5%3=2, 0, 1
    assert r.times[0].tolist() == [23.0, 24.0, 22.0]
    assert r.wp[0] == 8
    assert r.times[1].tolist() == [22.0, 23.0, 24.0] and r.wp[1] == 3


def test_key_collision_detection():
    assert O.key_collision(np.array([1.0, 2.0]), 4)       # M = 4 <= 7
    assert not O.key_collision(np.array([100.0]), 4)      # M = 102 > 7


def test_key_collision_changes_the_literal_rule():
    """With int(max t)+2 <= 2b-1 the reference key from*M+idx interleaves nodes;
    the literal restatement then departs from the lexicographic rule."""
    rng = np.random.default_rng(4)
    N, B, b, d = 3, 64, 150, 1
    (s, t_, tm, f), = _rand_batches(rng, N, 1, b, d, hot=1, t0=0.0)
    assert O.key_collision(tm, b)
    r1 = O.ring_advance(O.Ring.empty(N, B, d), s, t_, tm, f)
    r2 = O.ring_advance_brute(O.Ring.empty(N, B, d), s, t_, tm, f)
    assert not np.array_equal(r1.wp, r2.wp)


# ---------------------------------------------------------------- gather
def _rand_state(rng, N, B, d, with_csr):
    batches = _rand_batches(rng, N, 4, 25, d, hot=1)
    csr = None
    if with_csr:
        ev, eb = [], 0
        for (s, t_, tm, f) in batches[:2]:
            ev.append((s, t_, tm, f, eb))
            eb += len(s)
        csr = O.csr_freeze(N, d, ev)
        batches = batches[2:]
    ring = O.Ring.empty(N, B, d, with_eids=True)
    for (s, t_, tm, f) in batches:
        O.ring_advance(ring, s, t_, tm, f)
    return csr, ring, float(batches[-1][2][-1])


@pytest.mark.parametrize("seed,with_csr,K", [(0, False, 4), (1, True, 4), (2, True, 16), (3, False, 9)])
def test_recent_matches_bruteforce(seed, with_csr, K):
    rng = np.random.default_rng(seed)
    N, B, d = 9, 6, 2
    csr, ring, tmax = _rand_state(rng, N, B, d, with_csr)
    Q = 40
    nodes = rng.integers(-1, N, Q)
    qt = rng.uniform(90.0, tmax + 5.0, Q)
    qt[::9] = np.nan  # no entry is before a NaN time
    a = O.recent(nodes, qt, K, csr, ring, d)
    b = O.recent_brute(nodes, qt, K, csr, ring, d)
    for f in ("ids", "times", "feats", "mask", "eids"):
        assert np.array_equal(getattr(a, f), getattr(b, f)), f


def test_recent_known_answers_from_reference_tests():
    """tests/test_core.py:15-56 and tests/test_triton_kernel.py:76-117 restated (CSR path)."""
    d = 4
    ev = [(np.array([0, 0, 0, 1, 1]), np.array([1, 2, 3, 2, 3]),
           np.array([1.0, 2.0, 3.0, 1.5, 2.5]), np.zeros((5, d), np.float32), 0)]
    csr = O.csr_freeze(10, d, ev)
    r = O.recent(np.array([0]), np.array([4.0]), 3, csr, None, d)
    assert r.mask.all()
    ev = [(np.array([0, 0, 0]), np.array([1, 2, 3]), np.array([1.0, 5.0, 10.0]),
           np.zeros((3, 2), np.float32), 0)]
    csr = O.csr_freeze(5, 2, ev)
    r = O.recent(np.array([0]), np.array([6.0]), 3, csr, None, 2)
    assert r.ids[0].tolist() == [-1, 1, 2] and r.mask.sum() == 2
    ev = [(np.zeros(10, np.int64), np.arange(1, 11) % 10, np.arange(1, 11) * 0.1,
           np.zeros((10, 2), np.float32), 0)]
    csr = O.csr_freeze(10, 2, ev)
    r = O.recent(np.array([0]), np.array([0.55]), 10, csr, None, 2)
    assert r.mask.sum() == 5 and (r.times[r.mask] < 0.55).all()
    r = O.recent(np.array([-1, -1, 5]), np.array([0.5, 0.5, 0.5]), 8, csr, None, 2)
    assert (r.ids[:2] == -1).all() and r.mask[:2].sum() == 0


def test_ring_known_answer_async_ordering():
    """tests/test_async_pipeline.py:153-194: after a post-freeze advance of (1, 2, t=1),
    node 1's neighbours at t=2 contain 2."""
    ring = O.Ring.empty(10, 8, 2)
    O.ring_advance(ring, np.array([1]), np.array([2]), np.array([1.0]), np.zeros((1, 2), np.float32))
    r = O.recent(np.array([1]), np.array([2.0]), 8, O.CSR.empty(10, 2), ring, 2)
    assert 2 in r.ids[0].tolist()


def test_padding_query_reads_node0_ring_quirk():
    """With a ring, a query id < 0 reads node 0's ring (temporal_graph.py:312-319)."""
    ring = O.Ring.empty(4, 4, 1)
    O.ring_advance(ring, np.array([0]), np.array([3]), np.array([1.0]), np.ones((1, 1), np.float32))
    r = O.recent(np.array([-1]), np.array([5.0]), 2, O.CSR.empty(4, 1), ring, 1)
    assert r.ids[0].tolist() == [-1, 3]


# ---------------------------------------------------------------- time encoding
def test_time_weights_fixture():
    from pathlib import Path
    hexes = (Path(__file__).parent / "golden" / "time_weights_f32.txt").read_text().split()
    w = O.time_weights(100)
    assert [f"{v:08x}" for v in w.view(np.uint32)] == hexes
    assert w[0] == np.float32(1.0) and w[1] == np.float32(0.8111308) and w[99] == np.float32(1e-9)


def test_time_encode_closed_forms():
    w = O.time_weights(100)
    dt = np.array([[0.0, 1.0, 1e6]], np.float32)
    te = O.time_encode_exact(dt, w)
    assert np.all(te[0, 0] == 1.0)                      # cos(0) = 1 (self token t0)
    assert abs(te[0, 1, 0] - np.cos(1.0)) < 1e-15       # w0 = 1
    assert abs(te[0, 2, 99] - np.cos(np.float64(np.float32(np.float32(1e6) * np.float32(1e-9))))) < 1e-15
    m = np.array([[True, False, True]])
    assert np.all(O.time_encode_exact(dt, w, m)[0, 1] == 0.0)


def test_dt_conventions_differ_at_large_times():
    q = np.array([1e8 + 0.75])
    t = np.array([[1e8]])
    assert O.dt_dygformer(q, t)[0, 0] == np.float32(0.0)  # both round to the same fp32
    assert O.dt_tgn(q, t)[0, 0] == np.float32(0.75)


# ---------------------------------------------------------------- co-occurrence
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_co_occurrence_freq_matches_bruteforce(seed):
    rng = np.random.default_rng(seed)
    a = rng.integers(-1, 6, (7, 9))
    c = rng.integers(-1, 6, (7, 9))
    x1, y1 = O.co_occurrence_freq(a, c)
    x2, y2 = O.co_occurrence_freq_brute(a, c)
    assert np.array_equal(x1, x2) and np.array_equal(y1, y2)
    # (i) from (ii): pair count = #{i valid: a_cnt[i,1] > 0}
    pc = O.co_pair_count(a, a != -1, c, c != -1)
    assert np.array_equal(pc, ((a != -1) & (x1[..., 1] > 0)).sum(1).astype(np.float32))


@pytest.mark.parametrize("seed", [0, 1])
def test_co_occurrence_freq_masked(seed):
    rng = np.random.default_rng(seed)
    a = rng.integers(-1, 6, (7, 9))
    c = rng.integers(-1, 6, (7, 9))
    # masks ids != -1 reduce to the reference's id rule
    x, y = O.co_occurrence_freq_masked(a, a != -1, c, c != -1)
    x2, y2 = O.co_occurrence_freq(a, c)
    assert np.array_equal(x, x2) and np.array_equal(y, y2)
    # arbitrary masks: brute force over the valid positions only
    am = rng.random((7, 9)) < 0.6
    cm = rng.random((7, 9)) < 0.6
    x, y = O.co_occurrence_freq_masked(a, am, c, cm)
    for p in range(7):
        for i in range(9):
            ex = (sum(am[p, j] and a[p, j] == a[p, i] for j in range(9)),
                  sum(cm[p, j] and c[p, j] == a[p, i] for j in range(9))) if am[p, i] else (0, 0)
            ey = (sum(am[p, j] and a[p, j] == c[p, i] for j in range(9)),
                  sum(cm[p, j] and c[p, j] == c[p, i] for j in range(9))) if cm[p, i] else (0, 0)
            assert tuple(x[p, i]) == ex and tuple(y[p, i]) == ey
    # the pair count is #{valid i: a_cnt[i, 1] > 0} under the same masks
    assert np.array_equal(O.co_pair_count(a, am, c, cm), (am & (x[..., 1] > 0)).sum(1).astype(np.float32))


def test_co_pair_known_answers():
    """tests/test_core.py:59-76 (2), tests/test_cuda_kernels.py:225-263 (0 and 5)."""
    assert O.co_pair_count(np.array([[2, 3]]), np.array([[True, True]]),
                           np.array([[2, 3]]), np.array([[True, True]]))[0] == 2.0
    a = np.array([[1, 2, 3, 4, 5]])
    c = np.array([[12, 13, 14, 15, 16]])
    m = np.ones((1, 5), bool)
    assert O.co_pair_count(a, m, c, m)[0] == 0.0
    assert O.co_pair_count(a, m, a, m)[0] == 5.0


def test_co_dygformer_bruteforce_and_known_answers():
    rng = np.random.default_rng(3)
    A = rng.integers(-1, 5, (6, 8))
    C = rng.integers(-1, 5, (6, 8))
    af, cf = O.co_dygformer(A, C)
    for p in range(6):
        for i in range(8):
            ai, ci = A[p, i], C[p, i]
            ea = (0, 0) if ai == -1 else (int((A[p] == ai).sum()),
                                          int(((A[p] == ci) & (C[p] != -1)).sum()))
            ec = (0, 0) if ci == -1 else (int(((C[p] == ai) & (A[p] != -1)).sum()),
                                          int((C[p] == ci).sum()))
            assert tuple(af[p, i]) == ea and tuple(cf[p, i]) == ec
    # tests/test_dygformer.py:160-176: a repeated id counts itself twice
    af, _ = O.co_dygformer(np.array([[5, 5, 1, 2]]), np.array([[3, 4, 6, 7]]))
    assert af[0, 0, 0] == 2 and af[0, 1, 0] == 2 and af[0, 2, 0] == 1


# ---------------------------------------------------------------- planted mistakes
def _advance_time_order(ring, src, dst, time, feat, eid_base=0):
    """Plausible mistake: keep the B most recent entries (by time) instead of concat order."""
    B = ring.B
    frm, to, tt, ff = O._directed(src, dst, time, feat)
    for u in np.unique(frm):
        idx = np.flatnonzero(frm == u)
        idx = idx[np.argsort(tt[idx], kind="stable")][-B:]
        for m, e in enumerate(idx):
            s = (ring.wp[u] + m) % B
            ring.ids[u, s], ring.times[u, s], ring.feats[u, s] = to[e], tt[e], ff[e]
        ring.wp[u] += len(idx)
    return ring


def _advance_seq_ring(ring, src, dst, time, feat, eid_base=0):
    """Plausible mistake: a sequential ring (write_pos += c, not min(c, B))."""
    B = ring.B
    frm, to, tt, ff = O._directed(src, dst, time, feat)
    for u in np.unique(frm):
        idx = np.flatnonzero(frm == u)
        c = len(idx)
        for m, e in enumerate(idx[-B:]):
            s = (ring.wp[u] + (c - min(c, B)) + m) % B
            ring.ids[u, s], ring.times[u, s], ring.feats[u, s] = to[e], tt[e], ff[e]
        ring.wp[u] += c
    return ring


@pytest.mark.parametrize("mistake", [_advance_time_order, _advance_seq_ring])
def test_planted_ring_mistakes_are_caught(mistake):
    caught = False
    try:
        B = 2
        r = O.Ring.empty(5, B, 1)
        src = np.array([0, 0, 3], np.int64)
        dst = np.array([1, 2, 0], np.int64)
        time = np.array([1.0, 2.0, 0.5]) + 10.0
        mistake(r, src, dst, time, np.zeros((3, 1), np.float32))
        mistake(r, np.array([0]), np.array([4]), np.array([20.0]), np.zeros((1, 1), np.float32))
        assert r.ids[0].tolist() == [4, 3] and r.wp[0] == 3
        r2 = O.Ring.empty(2, 3, 1)
        r2.wp[0] = 5
        mistake(r2, np.zeros(5, np.int64), np.ones(5, np.int64), np.arange(5.0) + 20.0,
                np.zeros((5, 1), np.float32))
        assert r2.times[0].tolist() == [23.0, 24.0, 22.0] and r2.wp[0] == 8
    except AssertionError:
        caught = True
    assert caught, f"planted mistake {mistake.__name__} passed the ring checks"


def test_planted_gather_mistakes_are_caught():
    """Dropping the strict '<' (using '<='), or left-aligning, fails the known answers."""
    ev = [(np.array([0, 0, 0]), np.array([1, 2, 3]), np.array([1.0, 5.0, 10.0]),
           np.zeros((3, 2), np.float32), 0)]
    csr = O.csr_freeze(5, 2, ev)
    good = O.recent(np.array([0]), np.array([5.0]), 3, csr, None, 2)
    assert good.ids[0].tolist() == [-1, -1, 1]          # t=5 itself is excluded
    left = np.roll(good.ids[0], 2)
    assert left.tolist() != good.ids[0].tolist()
    le = [j for j in range(3) if ev[0][2][j] <= 5.0]
    assert len(le) != int(good.mask.sum())


def test_planted_cos_mistake_is_caught():
    """A dropped rounding of the fp32 argument (computing dt*w in float64) moves the
    encoding by more than the 1e-6 tolerance at large dt."""
    w = O.time_weights(100)
    dt = np.array([[3.7e7]], np.float32)
    exact = O.time_encode_exact(dt, w)
    wrong = np.cos(dt[..., None].astype(np.float64) * w.astype(np.float64))
    assert np.max(np.abs(exact - wrong)) > 1e-6


# ---------------------------------------------------------------- negative pool
def test_splitmix64_known_outputs():
    """mix64 is the splitmix64 finalizer: its outputs on the states G, 2G, 3G are
    the published first three values of splitmix64 seeded with 0."""
    G = 0x9E3779B97F4A7C15
    m = (1 << 64) - 1
    assert [O.mix64(k * G & m) for k in (1, 2, 3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                                      0x06C45D188009454F]
    assert O.uniform01(0) == 0.0 and O.uniform01(m) == np.float32(1 - 2.0 ** -24)


@pytest.mark.parametrize("P", [1, 4, 16])
def test_negpool_sorted_restatement_matches_sequential(P):
    """The device's two-sort formulation equals the edge-by-edge update, across the
    fill/replace boundary inside a batch, hot sources, same-slot collisions and
    out-of-range ids."""
    rng = np.random.default_rng(P)
    N = 30
    a = np.full((N, P), -1, np.int32)
    b = a.copy()
    ca = np.zeros(N, np.int64)
    cb = ca.copy()
    for call in range(12):
        n = int(rng.integers(0, 80))
        src = rng.integers(-1, N + 1, n)
        src[: n // 3] = 2  # a hot source
        dst = rng.integers(0, 1000, n)
        O.negpool_update(a, ca, src, dst, 77, call)
        O.negpool_update_sorted(b, cb, src, dst, 77, call)
        assert np.array_equal(a, b) and np.array_equal(ca, cb), call
    assert ca[2] > P  # the hot source went past the fill phase


def test_negpool_reservoir_keeps_every_edge_with_probability_p_over_n():
    """Reservoir sampling (negatives.py:45-53): after T edges of one source each
    edge is in the pool with probability P/T."""
    P, T, trials = 8, 64, 600
    hits = np.zeros(T)
    for seed in range(trials):
        pool = np.full((1, P), -1, np.int32)
        cnt = np.zeros(1, np.int64)
        for call, s in enumerate(range(0, T, 16)):
            O.negpool_update(pool, cnt, np.zeros(16, np.int64), np.arange(s, s + 16), seed, call)
        assert cnt[0] == T and (pool >= 0).all()
        hits[pool[0]] += 1
    p = hits / trials
    # each edge: binomial(600, 1/8), sd 0.0135; the mean is exact
    assert abs(p.mean() - P / T) < 1e-12
    assert np.abs(p - P / T).max() < 0.065
    assert abs(p[:T // 2].mean() - p[T // 2:].mean()) < 0.02  # old and new edges alike


def test_negpool_sample_is_uniform_over_valid_slots_and_falls_back():
    P, N = 16, 50
    pool = np.full((N, P), -1, np.int32)
    cnt = np.zeros(N, np.int64)
    pool[3, :5] = np.arange(100, 105)
    cnt[3] = 5
    out = O.negpool_sample(pool, cnt, np.full(5000, 3), 9, 0)
    vals, freq = np.unique(out, return_counts=True)
    assert list(vals) == list(range(100, 105))
    assert np.abs(freq / 5000 - 0.2).max() < 0.03
    fb = O.negpool_sample(pool, cnt, np.array([7, 7, 60, -1]), 9, 1)  # no history / out of range
    assert ((fb >= 0) & (fb < N)).all()


def test_negpool_draws_restatement_matches_the_counter_update():
    """negpool_update_draws (the reference's tensor formulation with its draws
    indexed by sorted position) equals the edge-by-edge update when handed the
    same draws, moved from batch order to sorted order; hot sources cross the
    fill/replace boundary and collide on slots."""
    rng = np.random.default_rng(5)
    N, P = 30, 4
    a = np.full((N, P), -1, np.int32)
    b = a.copy()
    ca = np.zeros(N, np.int64)
    cb = ca.copy()
    for call in range(15):
        n = int(rng.integers(1, 80))
        src = rng.integers(0, N, n)
        src[: n // 3] = 2
        dst = rng.integers(0, 1000, n)
        order = np.argsort(src, kind="stable")
        ua = np.array([O.uniform01(O.rand64(77, call, int(j), 0)) for j in order], np.float32)
        sd = np.array([O.rand64(77, call, int(j), 1) % P for j in order], np.int64)
        O.negpool_update(a, ca, src, dst, 77, call)
        O.negpool_update_draws(b, cb, src, dst, ua, sd)
        assert np.array_equal(a, b) and np.array_equal(ca, cb), call
        q = rng.integers(0, N, 50)
        us = np.array([O.uniform01(O.rand64(77, call, i, 2)) for i in range(50)], np.float32)
        want = O.negpool_sample(a, ca, q, 77, call)
        got = O.negpool_sample_draws(b, cb, q, us)
        hist = cb[q] > 0
        assert np.array_equal(got[hist], want[hist]) and (got[~hist] == -1).all()
    assert ca[2] > P


def test_negpool_draws_known_answers():
    """P = 2, one source, three edges in one batch: fill slots 0 and 1, then the
    third (e = 3) replaces slot_draw when u < f32(2) / f32(3) = 0.6666667."""
    for u, want in ((np.float32(0.66666657), [10, 12]), (np.float32(0.6666667), [10, 11]),
                    (np.float32(0.9), [10, 11])):
        pool = np.full((1, 2), -1, np.int32)
        cnt = np.zeros(1, np.int64)
        O.negpool_update_draws(pool, cnt, [0, 0, 0], [10, 11, 12], np.float32([0.0, 0.0, u]), [0, 0, 1])
        assert list(pool[0]) == want and cnt[0] == 3
    # sample: the 2 valid slots, int(u * 2); a row without history gives -1
    pool = np.array([[10, 11], [-1, -1]], np.int32)
    got = O.negpool_sample_draws(pool, np.array([2, 0]), [0, 0, 1], np.float32([0.49, 0.5, 0.3]))
    assert list(got) == [10, 11, -1]
