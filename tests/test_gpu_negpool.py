"""HistoricalNegPool on the device (tgx_negpool_update / tgx_negpool_sample)
against the oracle (the reference's reservoir update, edge by edge, with the
library's counter-based random numbers): pool slots, counts and samples bit for
bit after every call, on every update path (two launches with the cell table,
one workgroup, the sort), and the reservoir property measured on the device."""
import numpy as np
import pytest
import torch

from oracle import spec as O
from tgengine_amd.pipeline.negatives import HistoricalNegPool, HistoricalNegative

pytestmark = pytest.mark.gpu


def _check(pool, ref_pool, ref_cnt, where):
    assert np.array_equal(pool._pool.cpu().numpy(), ref_pool), f"{where}: pool"
    assert np.array_equal(pool._count.cpu().numpy(), ref_cnt), f"{where}: count"


class _NoScratch:
    """Stands in for the pool's cell table: the update then takes the paths that
    need none (one workgroup up to 8,192 edges, the sort above)."""

    def data_ptr(self):
        return 0

    def numel(self):
        return 0


def _pool(N, P, seed, scratch=True):
    pool = HistoricalNegPool(N, pool_size=P, device="cuda", seed=seed)
    if not scratch:
        pool._scratch = _NoScratch()
    return pool


@pytest.mark.parametrize("scratch", [True, False])
@pytest.mark.parametrize("N,P,b", [(40, 4, 90), (500, 16, 3000), (7, 1, 50), (2000, 512, 20000),
                                   (3000, 8, 40000)])
def test_negpool_matches_the_oracle(N, P, b, scratch):
    rng = np.random.default_rng(N + P)
    pool = _pool(N, P, 1234 + N, scratch)
    ref = np.full((N, P), -1, np.int32)
    cnt = np.zeros(N, np.int64)
    for call in range(8):
        n = int(rng.integers(1, b))
        src = rng.integers(0, N, n)
        src[: n // 3] = rng.integers(0, 3, n // 3)  # hot sources cross into replacement
        if call == 3:
            src[:5] = [-1, N, N + 7, -3, N]  # out of range: skipped
        dst = rng.integers(0, 10 * N, n)
        pool.update(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda())
        O.negpool_update(ref, cnt, src, dst, pool.seed, 2 * call)
        _check(pool, ref, cnt, f"update {call}")
        q = rng.integers(0, N, 400)
        q[:3] = [N - 1, 0, 1]
        got = pool.sample(torch.from_numpy(q).cuda()).cpu().numpy()
        exp = O.negpool_sample(ref, cnt, q, pool.seed, 2 * call + 1)
        assert np.array_equal(got, exp), f"sample {call}"
    assert cnt[:3].max() > P  # the hot sources went past the fill phase
    st = pool._status.cpu().numpy()
    assert st[0] == 5  # the five out-of-range sources of call 3


@pytest.mark.parametrize("scratch", [True, False])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 255, 256, 257, 1000, 1023, 1024, 1025, 4095, 4096, 4097, 5000,
                               8191, 8192, 8193, 12000, 32768, 32769])
def test_negpool_batch_sizes(n, scratch):
    """Batch sizes on both sides of the single-workgroup updates (at most 4,096 and
    8,192 edges, one thread per edge and round), of the two-launch update's
    workgroups (256 edges for batches of at most 256, else 1,024) and its limit
    (32,768 edges), and at a wavefront's boundary: three updates of n edges each,
    hot sources and a two-slot pool (many edges on one cell), pool and counts bit
    for bit after every call."""
    N, P = 64, 2
    rng = np.random.default_rng(n)
    pool = _pool(N, P, 99 + n, scratch)
    ref = np.full((N, P), -1, np.int32)
    cnt = np.zeros(N, np.int64)
    for call in range(3):
        src = rng.integers(0, N, n)
        src[: n // 2] = rng.integers(0, 2, n // 2)
        if n > 8:
            src[3] = -1
            src[7] = N
        dst = rng.integers(0, 1 << 30, n)
        pool.update(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda())
        O.negpool_update(ref, cnt, src, dst, pool.seed, 2 * call)
        _check(pool, ref, cnt, f"n={n} update {call}")
        pool._call += 1  # the sample call the reference stream would make


def test_negpool_empty_and_fresh_sources():
    pool = HistoricalNegPool(30, pool_size=8, device="cuda", seed=5)
    pool.update(torch.empty(0, dtype=torch.int64, device="cuda"), torch.empty(0, dtype=torch.int64, device="cuda"))
    out = pool.sample(torch.arange(30, device="cuda")).cpu().numpy()  # no history anywhere
    exp = O.negpool_sample(np.full((30, 8), -1, np.int32), np.zeros(30, np.int64), np.arange(30), 5, 1)
    assert np.array_equal(out, exp) and ((out >= 0) & (out < 30)).all()


def test_negpool_reservoir_property_on_device():
    """After T edges from one source, each edge sits in the pool with probability
    P/T (negatives.py:45-53); measured over 400 pools of different seeds."""
    P, T, trials, B = 16, 256, 400, 32
    hits = np.zeros(T)
    src = torch.zeros(B, dtype=torch.int64, device="cuda")
    for seed in range(trials):
        pool = HistoricalNegPool(1, pool_size=P, device="cuda", seed=seed)
        for s in range(0, T, B):
            pool.update(src, torch.arange(s, s + B, device="cuda"))
        row = pool._pool[0].cpu().numpy()
        assert (row >= 0).all() and len(set(row.tolist())) == P
        hits[row] += 1
    p = hits / trials
    # each edge: binomial(400, 1/16), sd 0.0121
    assert abs(p.mean() - P / T) < 1e-12
    assert np.abs(p - P / T).max() < 0.06
    assert abs(p[:T // 2].mean() - p[T // 2:].mean()) < 0.01


def test_historical_negative_strategy():
    strat = HistoricalNegative(100, pool_size=4, device="cuda", seed=3)
    src = torch.arange(10, device="cuda")
    strat.update(src, src + 50)
    neg = strat.sample(src, src + 50, None, None)
    assert torch.equal(neg, src + 50)  # one edge each: the only pool entry


@pytest.mark.parametrize("P,n", [(16, 300), (4, 5000), (8, 9000)])
def test_torch_rng_mode_reproduces_the_reference_draws(P, n):
    """rng="torch": the pool draws from torch's generator in the reference's call
    order and shapes (negatives.py:78-86, 116-124), so replaying the generator
    state into the oracle's draw-given restatement gives the same pool, counts
    and samples, and leaves the generator where the pool left it.  Batches on
    both sides of the single-workgroup update sizes; hot sources go past the
    fill phase."""
    rng = np.random.default_rng(40 + P)
    N = 500
    torch.manual_seed(1234)
    pool = HistoricalNegPool(N, P, device="cuda", rng="torch")
    cp = np.full((N, P), -1, np.int32)
    cc = np.zeros(N, np.int64)
    for step in range(6):
        src = rng.integers(0, N, n)
        src[: n // 4] = 7
        dst = rng.integers(0, N, n)
        state = torch.cuda.get_rng_state()
        pool.update(torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda())
        after = torch.cuda.get_rng_state()
        torch.cuda.set_rng_state(state)
        ua = torch.rand(n, device="cuda").cpu().numpy()
        sd = torch.randint(0, P, (n,), device="cuda").cpu().numpy()
        assert torch.equal(torch.cuda.get_rng_state(), after)
        O.negpool_update_draws(cp, cc, src, dst, ua, sd)
        assert np.array_equal(pool._pool.cpu().numpy(), cp), step
        assert np.array_equal(pool._count.cpu().numpy(), cc), step
        q = np.concatenate([rng.integers(0, N, 200), [N - 1, N - 2]])  # and nodes without history
        state = torch.cuda.get_rng_state()
        got = pool.sample(torch.from_numpy(q).cuda()).cpu().numpy()
        after = torch.cuda.get_rng_state()
        torch.cuda.set_rng_state(state)
        want = O.negpool_sample_draws(cp, cc, q, torch.rand(len(q), device="cuda").cpu().numpy())
        none = want < 0
        if none.any():
            want[none] = torch.randint(0, N, (int(none.sum()),), device="cuda").cpu().numpy()
        assert torch.equal(torch.cuda.get_rng_state(), after)
        assert np.array_equal(got, want), step
    assert cc[7] > P
