"""CPU oracle for the fused temporal data pipeline -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker.  The product path
(``tgengine_amd``) never imports it.

It restates, in numpy, the reference behaviour of ``tgengine`` for the hot path
(all paths relative to the reference checkout):

* ``ring_advance``        -- ``tgengine/core/temporal_graph.py:104-131`` (post-freeze
  branch) and ``_append_overflow`` ``:351-387``.
* ``ring_advance_brute``  -- the same rule written as a per-node loop (pins the above).
* ``csr_freeze``          -- ``freeze_csr`` ``:133-181``.
* ``recent``              -- ``recent`` ``:183-280`` with ``_gather_csr_window``
  ``:282-305`` and ``_merge_overflow`` ``:307-349``.
* ``recent_brute``        -- per-query brute force (pins the above).
* ``time_encode_*``       -- ``FixedCosineTimeEncoder`` (``tgengine/nn/time_encoding.py:37-63``)
  with the DyGFormer dt convention (``tgengine/models/dygformer.py:273-282``) and the
  TGN one (``tgengine/models/tgn.py:80``).
* ``co_occurrence_freq``  -- ``temporal_sample.cu:453-511`` (per-position counts).
* ``co_pair_count``       -- ``tgengine/pipeline/__init__.py:206-219``.
* ``co_dygformer``        -- ``tgengine/models/dygformer.py:71-87`` on ``1+K`` sequences.

Parity status of each function is listed in the repository's design notes; every
function here is pinned by a known-answer test, a brute-force twin or a closed
form in ``tests/test_oracle.py``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

PAD = -1

# fp32 frequencies of FixedCosineTimeEncoder: w = 1/10**linspace(0, 9, d) in fp32
# (tgengine/nn/time_encoding.py:49); bias is 0 (:52).


def time_weights(d_t: int = 100) -> np.ndarray:
    return (1.0 / (10 ** np.linspace(0, 9, d_t, dtype=np.float32))).astype(np.float32)


@dataclass
class Ring:
    """Per-node ring of ``B`` slots (temporal_graph.py:89-102)."""
    ids: np.ndarray      # (N, B) int32, -1 = empty
    times: np.ndarray    # (N, B) float64
    feats: np.ndarray    # (N, B, d) float32 (or uint16 bf16 bits)
    wp: np.ndarray       # (N,) int64
    eids: Optional[np.ndarray] = None  # (N, B) int64 edge ids (-1 = empty)

    @staticmethod
    def empty(N: int, B: int, d: int, feat_dtype=np.float32, with_eids: bool = False) -> "Ring":
        return Ring(ids=np.full((N, B), PAD, np.int32), times=np.zeros((N, B), np.float64),
                    feats=np.zeros((N, B, d), feat_dtype), wp=np.zeros(N, np.int64),
                    eids=np.full((N, B), -1, np.int64) if with_eids else None)

    def copy(self) -> "Ring":
        return Ring(self.ids.copy(), self.times.copy(), self.feats.copy(), self.wp.copy(),
                    None if self.eids is None else self.eids.copy())

    @property
    def B(self) -> int:
        return self.ids.shape[1]


def _directed(src, dst, time, feat):
    """advance(): one undirected event -> two directed entries (temporal_graph.py:125-128)."""
    frm = np.concatenate([src, dst]).astype(np.int64)
    to = np.concatenate([dst, src]).astype(np.int64)
    tt = np.concatenate([time, time]).astype(np.float64)
    ff = np.concatenate([feat, feat], axis=0)
    return frm, to, tt, ff


def key_collision(time: np.ndarray, b: int) -> bool:
    """True when ``from*(int(max t)+2)+idx`` is NOT a lexicographic key (temporal_graph.py:357)."""
    if len(time) == 0:
        return False
    M = int(float(np.max(time))) + 2
    return M <= 2 * b - 1


def ring_advance(ring: Ring, src, dst, time, feat, eid_base: int = 0) -> Ring:
    """Post-freeze advance: restates temporal_graph.py:123-129 and :351-387 step by step.

    key = from*M + arange(n), M = int(max t)+2; stable argsort; runs of equal
    ``from``; keep the last B entries of each run; slot = (wp + kept_offset) % B;
    wp += number kept.  Modifies ``ring`` in place and returns it.
    """
    b = len(src)
    if b == 0:
        return ring
    B = ring.B
    frm, to, tt, ff = _directed(src, dst, time, feat)
    n = 2 * b
    ev = np.concatenate([np.arange(b), np.arange(b)]).astype(np.int64) + eid_base
    M = int(float(tt.max())) + 2                                     # :357
    key = frm * M + np.arange(n, dtype=np.int64)
    perm = np.argsort(key, kind="stable")                            # :358
    s_from, s_to, s_t, s_f, s_ev = frm[perm], to[perm], tt[perm], ff[perm], ev[perm]
    # unique_consecutive (:365-367)
    head = np.ones(n, bool)
    head[1:] = s_from[1:] != s_from[:-1]
    run = np.cumsum(head) - 1
    starts = np.flatnonzero(head)
    cnts = np.diff(np.append(starts, n))
    off = np.arange(n) - starts[run]
    keep = off >= (cnts[run] - B)                                    # :369
    s_from, s_to, s_t, s_f, s_ev = s_from[keep], s_to[keep], s_t[keep], s_f[keep], s_ev[keep]
    nk = len(s_from)
    head2 = np.ones(nk, bool)
    head2[1:] = s_from[1:] != s_from[:-1]
    run2 = np.cumsum(head2) - 1
    starts2 = np.flatnonzero(head2)
    kept_off = np.arange(nk) - starts2[run2]                         # :376-378
    slot = (ring.wp[s_from] + kept_off) % B                          # :380
    ring.ids[s_from, slot] = s_to.astype(np.int32)                   # :382-384
    ring.times[s_from, slot] = s_t
    ring.feats[s_from, slot] = s_f
    if ring.eids is not None:
        ring.eids[s_from, slot] = s_ev
    np.add.at(ring.wp, s_from, 1)                                    # :386-387
    return ring


def ring_advance_brute(ring: Ring, src, dst, time, feat, eid_base: int = 0) -> Ring:
    """The same rule as a per-node loop over entries in concatenation order."""
    b = len(src)
    B = ring.B
    frm, to, tt, ff = _directed(src, dst, time, feat)
    per_node: dict = {}
    for i in range(2 * b):
        per_node.setdefault(int(frm[i]), []).append(i)
    for u, entries in per_node.items():
        kept = entries[-B:]
        for m, e in enumerate(kept):
            s = (int(ring.wp[u]) + m) % B
            ring.ids[u, s] = to[e]
            ring.times[u, s] = tt[e]
            ring.feats[u, s] = ff[e]
            if ring.eids is not None:
                ring.eids[u, s] = eid_base + (e % b)
        ring.wp[u] += len(kept)
    return ring


@dataclass
class CSR:
    """Frozen CSR (temporal_graph.py:133-181)."""
    offsets: np.ndarray  # (N+1,) int64
    ids: np.ndarray      # (E2,) int32
    times: np.ndarray    # (E2,) float64
    feats: np.ndarray    # (E2, d)
    eids: Optional[np.ndarray] = None

    @staticmethod
    def empty(N: int, d: int, feat_dtype=np.float32) -> "CSR":
        return CSR(np.zeros(N + 1, np.int64), np.zeros(0, np.int32), np.zeros(0, np.float64),
                   np.zeros((0, d), feat_dtype), np.zeros(0, np.int64))


def csr_freeze(N: int, d: int, events: list, feat_dtype=np.float32) -> CSR:
    """Build the CSR from pre-freeze advance() calls.

    ``events`` is a list of (src, dst, time, feat, eid_base) tuples in call order.
    Build order per call is [src->dst for each event, dst->src for each event]
    (temporal_graph.py:110-122); the build sorts stably by time, then stably by
    node (:156-158), so within a node entries are time-ascending, ties in build order.
    """
    frm_l, to_l, t_l, f_l, e_l = [], [], [], [], []
    for (src, dst, time, feat, eb) in events:
        b = len(src)
        frm_l += [src, dst]
        to_l += [dst, src]
        t_l += [time, time]
        f_l += [feat, feat]
        ev = np.arange(b, dtype=np.int64) + eb
        e_l += [ev, ev]
    if not frm_l or sum(len(x) for x in frm_l) == 0:
        return CSR.empty(N, d, feat_dtype)
    frm = np.concatenate(frm_l).astype(np.int64)
    to = np.concatenate(to_l).astype(np.int32)
    tt = np.concatenate(t_l).astype(np.float64)
    ff = np.concatenate(f_l, axis=0)
    ee = np.concatenate(e_l)
    perm = np.argsort(tt, kind="stable")
    perm = perm[np.argsort(frm[perm], kind="stable")]
    counts = np.bincount(frm, minlength=N).astype(np.int64)
    offsets = np.zeros(N + 1, np.int64)
    offsets[1:] = np.cumsum(counts)
    return CSR(offsets, to[perm], tt[perm], ff[perm], ee[perm])


@dataclass
class Neighbors:
    ids: np.ndarray    # (Q, K) int32
    times: np.ndarray  # (Q, K) float64
    feats: np.ndarray  # (Q, K, d)
    mask: np.ndarray   # (Q, K) bool
    eids: Optional[np.ndarray] = None  # (Q, K) int64


def recent(nodes, qtimes, K: int, csr: Optional[CSR], ring: Optional[Ring], d: int,
           feat_dtype=np.float32) -> Neighbors:
    """recent() as the reference evaluates it (temporal_graph.py:183-349).

    CSR window: count = #{t < q} by lower bound, take = min(count, K), right
    aligned (:241-305); padding queries (id < 0) get an empty window (:233-235).
    A NaN query time counts no entry (the reference's searchsorted over rows
    padded with +inf returns the padded row length there, so its window would
    run past the node's own entries: no defined answer to restate).
    Ring merge (:307-349): ring rows of max(node, 0) -- a padding query reads
    node 0's ring -- valid = id != -1 and t < q; candidates = K CSR slots ++ B
    ring slots, keyed by time (-inf when invalid), ascending, last K kept.
    Ties between valid candidates keep CSR-before-ring then slot order (the
    reference sort is unstable there; see the module docstring of tests).
    """
    nodes = np.asarray(nodes, np.int64)
    qtimes = np.asarray(qtimes, np.float64)
    Q = len(nodes)
    out_ids = np.full((Q, K), PAD, np.int32)
    out_t = np.zeros((Q, K), np.float64)
    out_f = np.zeros((Q, K, d), feat_dtype)
    out_m = np.zeros((Q, K), bool)
    out_e = np.full((Q, K), -1, np.int64)
    if Q == 0:
        return Neighbors(out_ids, out_t, out_f, out_m, out_e)
    # --- CSR part
    if csr is not None and len(csr.ids) > 0:
        safe = np.maximum(nodes, 0)
        st = csr.offsets[safe].copy()
        en = csr.offsets[safe + 1].copy()
        pad = nodes < 0
        st[pad] = 0
        en[pad] = 0
        for q in range(Q):
            seg = csr.times[st[q]:en[q]]
            # #{t < q}: NaN entries sort last and never count; a NaN query time
            # counts none (searchsorted would place it after every entry)
            cnt = 0 if np.isnan(qtimes[q]) else int(np.searchsorted(seg, qtimes[q], side="left"))
            take = min(cnt, K)
            lo = st[q] + cnt - take
            out_ids[q, K - take:] = csr.ids[lo:lo + take]
            out_t[q, K - take:] = csr.times[lo:lo + take]
            out_f[q, K - take:] = csr.feats[lo:lo + take]
            out_m[q, K - take:] = True
            if csr.eids is not None:
                out_e[q, K - take:] = csr.eids[lo:lo + take]
    if ring is None:
        return Neighbors(out_ids, out_t, out_f, out_m, out_e)
    # --- ring merge
    safe = np.maximum(nodes, 0)
    r_ids = ring.ids[safe]
    r_t = ring.times[safe]
    r_f = ring.feats[safe]
    r_e = ring.eids[safe] if ring.eids is not None else np.full(r_ids.shape, -1, np.int64)
    r_valid = (r_ids != PAD) & (r_t < qtimes[:, None])
    if not r_valid.any():
        return Neighbors(out_ids, out_t, out_f, out_m, out_e)
    a_ids = np.concatenate([out_ids, r_ids], axis=1)
    a_t = np.concatenate([out_t, r_t], axis=1)
    a_f = np.concatenate([out_f, r_f], axis=1)
    a_m = np.concatenate([out_m, r_valid], axis=1)
    a_e = np.concatenate([out_e, r_e], axis=1)
    key = np.where(a_m, a_t, -np.inf)
    order = np.argsort(key, axis=1, kind="stable")
    sel = order[:, -K:]
    rows = np.arange(Q)[:, None]
    ids = a_ids[rows, sel]
    t = a_t[rows, sel]
    f = a_f[rows, sel]
    m = a_m[rows, sel]
    e = a_e[rows, sel]
    # invalid candidates chosen as padding: canonical pad values (under strictly
    # increasing streams every invalid candidate already is (-1, 0.0, 0, False))
    ids = np.where(m, ids, PAD).astype(np.int32)
    t = np.where(m, t, 0.0)
    f = np.where(m[..., None], f, np.zeros((), f.dtype)).astype(feat_dtype)
    e = np.where(m, e, -1)
    return Neighbors(ids, t, f, m, e)


def recent_brute(nodes, qtimes, K: int, csr: Optional[CSR], ring: Optional[Ring], d: int,
                 feat_dtype=np.float32) -> Neighbors:
    """Per-query brute force: collect every valid candidate, sort by (time, source order)."""
    Q = len(nodes)
    out = Neighbors(np.full((Q, K), PAD, np.int32), np.zeros((Q, K)),
                    np.zeros((Q, K, d), feat_dtype), np.zeros((Q, K), bool),
                    np.full((Q, K), -1, np.int64))
    for q in range(Q):
        u = int(nodes[q])
        tq = float(qtimes[q])
        cand = []  # (time, order, id, feat, eid)
        if csr is not None and len(csr.ids) > 0 and u >= 0:
            lo, hi = int(csr.offsets[u]), int(csr.offsets[u + 1])
            idx = [j for j in range(lo, hi) if csr.times[j] < tq][-K:]
            for o, j in enumerate(idx):
                cand.append((csr.times[j], o, int(csr.ids[j]), csr.feats[j],
                             int(csr.eids[j]) if csr.eids is not None else -1))
        if ring is not None:
            ur = max(u, 0)
            for s in range(ring.B):
                if ring.ids[ur, s] != PAD and ring.times[ur, s] < tq:
                    cand.append((ring.times[ur, s], K + s, int(ring.ids[ur, s]), ring.feats[ur, s],
                                 int(ring.eids[ur, s]) if ring.eids is not None else -1))
        cand.sort(key=lambda c: (c[0], c[1]))
        cand = cand[-K:]
        V = len(cand)
        for p, c in enumerate(cand):
            out.ids[q, K - V + p] = c[2]
            out.times[q, K - V + p] = c[0]
            out.feats[q, K - V + p] = c[3]
            out.mask[q, K - V + p] = True
            out.eids[q, K - V + p] = c[4]
    return out


# ---------------------------------------------------------------------------
# time encoding
# ---------------------------------------------------------------------------

def dt_dygformer(qtimes, nbr_times) -> np.ndarray:
    """dt32 = f32(q) - f32(t) in fp32 (dygformer.py:274-275)."""
    q = np.asarray(qtimes, np.float64).astype(np.float32)
    t = np.asarray(nbr_times, np.float64).astype(np.float32)
    return (q[:, None] - t).astype(np.float32)


def dt_tgn(qtimes, nbr_times) -> np.ndarray:
    """dt32 = f32(q - t) with the subtraction in float64 (tgn.py:80, time_encoding.py:63)."""
    q = np.asarray(qtimes, np.float64)
    return (q[:, None] - np.asarray(nbr_times, np.float64)).astype(np.float32)


def time_args(dt32: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """fp32 argument fl32(dt*w) (+ bias, rounded again) for every (…, j)."""
    a = (dt32[..., None].astype(np.float32) * w.astype(np.float32)).astype(np.float32)
    if bias is not None:
        a = (a + bias.astype(np.float32)).astype(np.float32)
    return a


def time_encode_exact(dt32: np.ndarray, w: np.ndarray, mask: Optional[np.ndarray] = None,
                      bias: Optional[np.ndarray] = None) -> np.ndarray:
    """cos of the exact fp32 argument, in float64; zero where ``mask`` is False."""
    te = np.cos(time_args(dt32, w, bias).astype(np.float64))
    if mask is not None:
        te = np.where(mask[..., None], te, 0.0)
    return te


# ---------------------------------------------------------------------------
# co-occurrence
# ---------------------------------------------------------------------------

def co_occurrence_freq(a: np.ndarray, c: np.ndarray):
    """Per position counts (temporal_sample.cu:453-511), int32.

    a_cnt[p,i] = (#{j: a[j]==a[i]}, #{j: c[j]==a[i]}), c_cnt[p,i] = (#{j: a[j]==c[i]},
    #{j: c[j]==c[i]}); both (0, 0) at padding ids (-1).
    """
    a = np.asarray(a, np.int64)
    c = np.asarray(c, np.int64)
    aa = (a[:, :, None] == a[:, None, :]).sum(-1)
    ac = (a[:, :, None] == c[:, None, :]).sum(-1)
    ca = (c[:, :, None] == a[:, None, :]).sum(-1)
    cc = (c[:, :, None] == c[:, None, :]).sum(-1)
    a_cnt = np.stack([aa, ac], -1).astype(np.int32)
    c_cnt = np.stack([ca, cc], -1).astype(np.int32)
    a_cnt[a == PAD] = 0
    c_cnt[c == PAD] = 0
    return a_cnt, c_cnt


def co_occurrence_freq_brute(a, c):
    P, K = a.shape
    a_cnt = np.zeros((P, K, 2), np.int32)
    c_cnt = np.zeros((P, K, 2), np.int32)
    for p in range(P):
        for i in range(K):
            if a[p, i] != PAD:
                a_cnt[p, i, 0] = sum(1 for j in range(K) if a[p, j] == a[p, i])
                a_cnt[p, i, 1] = sum(1 for j in range(K) if c[p, j] == a[p, i])
            if c[p, i] != PAD:
                c_cnt[p, i, 0] = sum(1 for j in range(K) if a[p, j] == c[p, i])
                c_cnt[p, i, 1] = sum(1 for j in range(K) if c[p, j] == c[p, i])
    return a_cnt, c_cnt


def co_occurrence_freq_masked(a, a_mask, c, c_mask):
    """Per-position counts over the valid positions only (tgx_co_occurrence with
    masks): a_cnt[p,i] = (#{j valid in a: a[j]==a[i]}, #{j valid in c: c[j]==a[i]})
    at a valid position i, (0, 0) elsewhere; c_cnt likewise.  With masks
    ``ids != -1`` this is co_occurrence_freq (temporal_sample.cu:453-511)."""
    a = np.asarray(a, np.int64)
    c = np.asarray(c, np.int64)
    am = np.asarray(a_mask, bool)
    cm = np.asarray(c_mask, bool)
    aa = ((a[:, :, None] == a[:, None, :]) & am[:, None, :]).sum(-1)
    ac = ((a[:, :, None] == c[:, None, :]) & cm[:, None, :]).sum(-1)
    ca = ((c[:, :, None] == a[:, None, :]) & am[:, None, :]).sum(-1)
    cc = ((c[:, :, None] == c[:, None, :]) & cm[:, None, :]).sum(-1)
    a_cnt = np.stack([aa, ac], -1).astype(np.int32)
    c_cnt = np.stack([ca, cc], -1).astype(np.int32)
    a_cnt[~am] = 0
    c_cnt[~cm] = 0
    return a_cnt, c_cnt


def co_pair_count(a_ids, a_mask, c_ids, c_mask) -> np.ndarray:
    """(P,) float32: #{i: a valid and some valid c[j]==a[i]} (pipeline/__init__.py:206-219)."""
    eq = a_ids[:, :, None] == c_ids[:, None, :]
    valid = a_mask[:, :, None] & c_mask[:, None, :]
    return (eq & valid).any(axis=2).astype(np.float32).sum(axis=1)


def co_dygformer(a_full, c_full):
    """DyGFormer in-model counts on 1+K sequences (dygformer.py:71-87), int32.

    a_freq[i] = (#{j: A[j]==A[i]}, #{j: A[j]==C[i], C[j]!=pad}) with padding masks as in
    the broadcast form; c_freq symmetric with the cross channel first.
    """
    A = np.asarray(a_full, np.int64)
    C = np.asarray(c_full, np.int64)
    a_pad = A == PAD
    c_pad = C == PAD
    a_self = (A[:, None, :] == A[:, :, None]).astype(np.int32)   # [b, i, j] = A[j]==A[i]
    c_self = (C[:, None, :] == C[:, :, None]).astype(np.int32)
    cross = (A[:, None, :] == C[:, :, None]).astype(np.int32)    # [b, i, j] = A[j]==C[i]
    a_self[a_pad[:, :, None] | a_pad[:, None, :]] = 0
    c_self[c_pad[:, :, None] | c_pad[:, None, :]] = 0
    cross[a_pad[:, :, None] | c_pad[:, None, :]] = 0
    a_freq = np.stack([a_self.sum(1), cross.sum(2)], axis=2)
    c_freq = np.stack([cross.sum(1), c_self.sum(1)], axis=2)
    return a_freq.astype(np.int32), c_freq.astype(np.int32)


# ---------------------------------------------------------------- negative pool
# HistoricalNegPool (reference pipeline/negatives.py:14-126) with the library's
# counter-based random numbers in place of torch.rand / torch.randint.

_M64 = (1 << 64) - 1
_GOLDEN = 0x9E3779B97F4A7C15


def mix64(z: int) -> int:
    """The splitmix64 finalizer (Steele, Lea, Flood 2014; Vigna's splitmix64.c)."""
    z &= _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def rand64(seed: int, call: int, i: int, stream: int) -> int:
    return mix64(mix64(mix64((seed ^ _GOLDEN) & _M64) ^ (call & _M64)) ^ ((4 * i + stream) & _M64))


def uniform01(h: int) -> np.float32:
    return np.float32(h >> 40) * np.float32(2.0 ** -24)


def negpool_update(pool: np.ndarray, count: np.ndarray, src, dst, seed: int, call: int) -> None:
    """One update, edge by edge in batch order (negatives.py:45-103): edge j, the
    r-th of its source u in the batch, is u's e-th edge, e = count[u] + r + 1
    (count from before the batch); e <= P fills slot e-1, else it replaces slot
    rand % P with probability P/e in float32.  Sequential writes: a later edge
    overwrites an earlier one's slot.  count[u] grows by u's edges."""
    N, P = pool.shape
    seen: dict = {}
    for j in range(len(src)):
        u = int(src[j])
        if u < 0 or u >= N:
            continue
        r = seen.get(u, 0)
        seen[u] = r + 1
        e = int(count[u]) + r + 1
        if e <= P:
            slot = e - 1
        elif uniform01(rand64(seed, call, j, 0)) < np.float32(P) / np.float32(e):
            slot = rand64(seed, call, j, 1) % P
        else:
            continue
        pool[u, slot] = np.int32(dst[j])
    for u, c in seen.items():
        count[u] += c


def negpool_update_sorted(pool: np.ndarray, count: np.ndarray, src, dst, seed: int, call: int) -> None:
    """The same update as the device computes it: a stable sort by source gives
    r, a stable sort of accepted edges by (u, slot) keeps the latest per slot."""
    N, P = pool.shape
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    n = len(src)
    ok = (src >= 0) & (src < N)
    idx = np.nonzero(ok)[0]
    order = idx[np.argsort(src[idx], kind="stable")]
    su = src[order]
    start = np.searchsorted(su, su, side="left")
    r = np.arange(len(order)) - start
    e = count[su] + r + 1
    keys, vals = [], []
    for p in range(len(order)):
        j = int(order[p])
        if e[p] <= P:
            slot = int(e[p]) - 1
        elif uniform01(rand64(seed, call, j, 0)) < np.float32(P) / np.float32(e[p]):
            slot = rand64(seed, call, j, 1) % P
        else:
            continue
        keys.append(int(su[p]) * P + slot)
        vals.append(j)
    keys = np.asarray(keys, np.int64)
    vals = np.asarray(vals, np.int64)
    o = np.argsort(keys, kind="stable")
    keys, vals = keys[o], vals[o]
    last = np.ones(len(keys), bool)
    last[:-1] = keys[1:] != keys[:-1]
    pool.reshape(-1)[keys[last]] = dst[vals[last]].astype(np.int32)
    np.add.at(count, su, 1)


def negpool_sample(pool: np.ndarray, count: np.ndarray, src, seed: int, call: int) -> np.ndarray:
    """negatives.py:105-126: a uniform slot among the valid ones (a prefix of
    min(count, P) slots), int(f32(U) * f32(v)) clamped to P-1; a random node when
    the source has no history."""
    N, P = pool.shape
    out = np.empty(len(src), np.int64)
    for q in range(len(src)):
        u = int(src[q])
        c = int(count[u]) if 0 <= u < N else 0
        v = min(c, P)
        if v > 0:
            s = min(int(uniform01(rand64(seed, call, q, 2)) * np.float32(v)), P - 1)
            out[q] = pool[u, s]
        else:
            out[q] = rand64(seed, call, q, 3) % N
    return out


def negpool_update_draws(pool: np.ndarray, count: np.ndarray, src, dst, u_accept, slot_draw) -> None:
    """negatives.py:45-103 with the draws given as the reference takes them:
    ``u_accept`` (torch.rand(n)) and ``slot_draw`` (torch.randint(0, P, (n,)))
    indexed by the edge's position in the stable argsort of src.  Position p,
    the r-th edge of its source u, is u's e-th edge, e = count[u] + r + 1: e <= P
    fills slot e - 1; otherwise u_accept[p] < f32(P) / f32(e) replaces slot
    slot_draw[p].  The accepted edges are written in sorted order (a later write
    of one (u, slot) wins), and count[u] grows by u's edges."""
    N, P = pool.shape
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    n = len(src)
    if n == 0:
        return
    order = np.argsort(src, kind="stable")
    su, sd = src[order], dst[order]
    start = np.searchsorted(su, su, side="left")
    r = np.arange(n) - start
    e = count[su] + r + 1
    fill = e <= P
    ua = np.asarray(u_accept, np.float32)
    replace = ~fill & (ua < np.float32(P) / e.astype(np.float32))
    slot = np.where(fill, np.minimum(e - 1, P - 1), np.asarray(slot_draw, np.int64))
    acc = fill | replace
    for p in np.nonzero(acc)[0]:  # in sorted order: the later write stays
        pool[su[p], slot[p]] = np.int32(sd[p])
    np.add.at(count, su, 1)


def negpool_sample_draws(pool: np.ndarray, count: np.ndarray, src, u_slot) -> np.ndarray:
    """negatives.py:105-126 with torch.rand(B) given as ``u_slot``: among the
    valid (non-padding) slots of the source's pool row, slot int(f32(U) *
    f32(valid)) clamped to P - 1; -1 where the row holds no valid slot (the
    reference fills those with torch.randint(0, N, (k,)) in query order)."""
    N, P = pool.shape
    src = np.asarray(src, np.int64)
    rows = pool[src]
    valid = (rows != -1).sum(1)
    idx = (np.asarray(u_slot, np.float32) * valid.astype(np.float32)).astype(np.int64)
    idx = np.minimum(idx, P - 1)
    out = rows[np.arange(len(src)), idx].astype(np.int64)
    out[valid == 0] = -1
    return out
