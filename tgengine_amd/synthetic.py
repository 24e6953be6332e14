"""Seeded synthetic event streams for the five benchmark configurations.

Every batch is drawn from its own PCG64 substream
(``SeedSequence(config.seed, spawn_key=(batch_index,))``), so any window of a
stream can be regenerated on its own and the GPU path, the CPU oracle and the
CPU baseline all see the same bytes.

Time model: batch ``i`` owns the window ``[t0 + i*L, t0 + (i+1)*L)`` with
``L = batch * mean_gap``.  Inside the window the ``b`` event times are the
normalised cumulative sums of ``b+1`` positive gaps drawn from the configured
inter-arrival law (exponential, or a two-component exponential mixture for the
bursty stream).  Times are then forced strictly increasing with ``nextafter``,
so no two events share a timestamp.  ``t0 = 2*batch`` keeps the reference's
ring sort key ``from*(int(max_t)+2)+idx`` collision free for every batch
(``int(max_t)+2 > 2*batch - 1``).

Degree laws: ``zipf(a)`` is the truncated Zipf law ``P(rank k) ~ k**-a`` over
the id range, mapped rank -> id through a fixed seeded permutation.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from functools import lru_cache
from typing import Optional

import numpy as np

__all__ = ["StreamConfig", "CONFIGS", "ENGINE_SHAPES", "gen_batch", "num_batches", "f32_to_bf16_bits",
           "bf16_bits_to_f32", "make_graph", "make_pipeline", "to_raw"]


@dataclass(frozen=True)
class StreamConfig:
    name: str
    num_nodes: int
    num_events: int
    # id ranges [lo, hi) for src and dst draws
    src_range: tuple
    dst_range: tuple
    src_law: str            # "uniform" | "zipf"
    dst_law: str
    src_a: float = 0.0
    dst_a: float = 0.0
    shared_perm: bool = True   # src and dst zipf ranks use one rank->id map
    feat_dim: int = 172
    feat_dtype: str = "f32"    # "f32" | "bf16"
    buffer_size: int = 32
    batch: int = 200
    k: int = 20
    n_neg: int = 1             # negatives per positive (1 -> neg is (b,))
    co_occurrence: bool = False
    time_law: str = "exp"      # "exp" | "bursty"
    mean_gap: float = 1.0
    burst_scales: tuple = (0.01, 10.0)
    burst_weight: float = 0.5  # probability of the short-gap component
    hot_nodes: int = 0         # extra hot nodes (each ~hot_share of events)
    hot_share: float = 0.01
    seed: int = 0
    d_t: int = 100

    @property
    def queries_per_event(self) -> int:
        return 2 + self.n_neg

    @property
    def feat_bytes(self) -> int:
        return 4 if self.feat_dtype == "f32" else 2


CONFIGS = {
    # C1: Wikipedia-like bipartite stream (reference CPU-runnable case)
    "c1": StreamConfig("c1", 9227, 157_474, (0, 8227), (8227, 9227), "uniform", "zipf",
                       dst_a=1.1, feat_dim=172, feat_dtype="f32", buffer_size=32, batch=200,
                       k=20, seed=1001),
    # C2: skewed one-id-space stream with co-occurrence
    "c2": StreamConfig("c2", 10984, 672_447, (0, 10984), (0, 10984), "zipf", "zipf",
                       src_a=1.2, dst_a=1.2, feat_dim=172, feat_dtype="f32", buffer_size=32,
                       batch=200, k=32, co_occurrence=True, seed=1002),
    # C3: large sparse stream, bf16 16-d features, hot nodes
    "c3": StreamConfig("c3", 1_000_000, 50_000_000, (0, 1_000_000), (0, 1_000_000), "zipf",
                       "zipf", src_a=1.5, dst_a=1.5, feat_dim=16, feat_dtype="bf16",
                       buffer_size=32, batch=4000, k=20, hot_nodes=4, hot_share=0.01,
                       seed=1003),
    # C4: feature-heavy stream, 512-d bf16, 5 negatives
    "c4": StreamConfig("c4", 100_000, 10_000_000, (0, 100_000), (0, 100_000), "uniform", "zipf",
                       dst_a=1.1, feat_dim=512, feat_dtype="bf16", buffer_size=64, batch=2000,
                       k=64, n_neg=5, seed=1004),
    # C5: full DyGFormer-style prepare pass, bursty times, co-occurrence
    "c5": StreamConfig("c5", 2_000_000, 100_000_000, (0, 2_000_000), (0, 2_000_000), "zipf",
                       "zipf", src_a=1.3, dst_a=1.3, feat_dim=172, feat_dtype="f32",
                       buffer_size=32, batch=8192, k=32, co_occurrence=True, time_law="bursty",
                       seed=1005),
}


# The shapes of the reference's published pipeline timings (Engine on a frozen CSR,
# batch 200, docs/performance_report.md:29-31): node and event counts, bipartite
# id ranges, K and edge-feature width of Wikipedia, Reddit and LastFM, as
# synthetic streams (the datasets themselves are not available here)
ENGINE_SHAPES = {
    "wikipedia": StreamConfig("wikipedia", 9228, 157_474, (0, 8228), (8228, 9228), "uniform", "zipf",
                              dst_a=1.1, feat_dim=172, feat_dtype="f32", batch=200, k=32, seed=2001),
    "reddit": StreamConfig("reddit", 10985, 672_447, (0, 10000), (10000, 10985), "zipf", "zipf",
                           src_a=1.1, dst_a=1.1, feat_dim=172, feat_dtype="f32", batch=200, k=64,
                           seed=2002),
    "lastfm": StreamConfig("lastfm", 1981, 1_293_103, (0, 980), (980, 1981), "zipf", "zipf",
                           src_a=0.8, dst_a=1.0, feat_dim=2, feat_dtype="f32", batch=200, k=512,
                           seed=2003),
}


def num_batches(cfg: StreamConfig) -> int:
    return (cfg.num_events + cfg.batch - 1) // cfg.batch


def batch_len(cfg: StreamConfig, i: int) -> int:
    return min(cfg.batch, cfg.num_events - i * cfg.batch)


def _window(cfg: StreamConfig) -> float:
    if cfg.time_law == "bursty":
        s0, s1 = cfg.burst_scales
        mean = cfg.burst_weight * s0 + (1.0 - cfg.burst_weight) * s1
    else:
        mean = cfg.mean_gap
    return cfg.batch * mean


def t0(cfg: StreamConfig) -> float:
    return float(2 * cfg.batch)


@lru_cache(maxsize=16)
def _zipf_cdf(n: int, a: float) -> np.ndarray:
    k = np.arange(1, n + 1, dtype=np.float64)
    p = k ** (-a)
    c = np.cumsum(p)
    c /= c[-1]
    c[-1] = 1.0
    return c


@lru_cache(maxsize=16)
def _rank_perm(seed: int, lo: int, hi: int, tag: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence(seed, spawn_key=(1 << 40, tag))))
    return (lo + rng.permutation(hi - lo)).astype(np.int64)


def _draw(rng: np.random.Generator, cfg: StreamConfig, law: str, a: float, rng_ids: tuple,
          b: int, tag: int) -> np.ndarray:
    lo, hi = rng_ids
    if law == "uniform":
        return rng.integers(lo, hi, size=b, dtype=np.int64)
    cdf = _zipf_cdf(hi - lo, a)
    r = np.searchsorted(cdf, rng.random(b), side="right")
    r = np.minimum(r, hi - lo - 1)
    perm = _rank_perm(cfg.seed, lo, hi, 0 if cfg.shared_perm else tag)
    return perm[r]


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return ((u + rounding) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << np.uint32(16)).view(np.float32)


def gen_batch(cfg: StreamConfig, i: int, with_feats: bool = True) -> dict:
    """Batch ``i`` of stream ``cfg`` as numpy arrays.

    Returns ``src, dst`` int64 (b,), ``time`` float64 (b,), ``feat`` (b, d)
    float32 or uint16 bf16 bits, ``neg`` int64 (b,) or (b, n_neg).
    """
    b = batch_len(cfg, i)
    if b <= 0:
        raise IndexError(f"batch {i} out of range for {cfg.name}")
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence(cfg.seed, spawn_key=(i,))))
    src = _draw(rng, cfg, cfg.src_law, cfg.src_a, cfg.src_range, b, 1)
    dst = _draw(rng, cfg, cfg.dst_law, cfg.dst_a, cfg.dst_range, b, 2)
    if cfg.hot_nodes > 0:
        hot_ids = _rank_perm(cfg.seed, 0, cfg.num_nodes, 3)[:cfg.hot_nodes]
        u = rng.random(b)
        which = rng.integers(0, cfg.hot_nodes, size=b)
        side = rng.random(b) < 0.5
        is_hot = u < cfg.hot_nodes * cfg.hot_share
        src = np.where(is_hot & side, hot_ids[which], src)
        dst = np.where(is_hot & ~side, hot_ids[which], dst)
    # times
    if cfg.time_law == "bursty":
        s0, s1 = cfg.burst_scales
        pick = rng.random(b + 1) < cfg.burst_weight
        gaps = np.where(pick, rng.exponential(s0, b + 1), rng.exponential(s1, b + 1))
    else:
        gaps = rng.exponential(cfg.mean_gap, b + 1)
    gaps = np.maximum(gaps, 1e-300)
    c = np.cumsum(gaps)
    L = _window(cfg)
    time = t0(cfg) + i * L + L * (c[:b] / c[b])
    if b > 1 and np.any(np.diff(time) <= 0):  # strict increase (rarely needed)
        for k in range(1, b):
            if time[k] <= time[k - 1]:
                time[k] = np.nextafter(time[k - 1], np.inf)
    if with_feats:
        f = rng.standard_normal((b, cfg.feat_dim), dtype=np.float32)
        feat = f if cfg.feat_dtype == "f32" else f32_to_bf16_bits(f)
    else:
        feat = None
    if cfg.n_neg == 1:
        neg = rng.integers(0, cfg.num_nodes, size=b, dtype=np.int64)
    else:
        neg = rng.integers(0, cfg.num_nodes, size=(b, cfg.n_neg), dtype=np.int64)
    return {"src": src, "dst": dst, "time": time, "feat": feat, "neg": neg}


def key_multiplier_ok(time: np.ndarray, b: int) -> bool:
    """True when the reference ring sort key is a lexicographic (node, index) key."""
    M = int(float(np.max(time))) + 2
    return M > 2 * b - 1


def make_graph(cfg: StreamConfig, device="cuda", track_edge_ids: bool = False):
    """An empty TemporalGraph laid out for ``cfg`` (ring of cfg.buffer_size slots,
    the config's feature width and storage dtype)."""
    import torch
    from tgengine_amd import TemporalGraph
    return TemporalGraph(cfg.num_nodes, edge_feat_dim=cfg.feat_dim, device=device,
                         buffer_size=cfg.buffer_size,
                         feat_dtype=torch.bfloat16 if cfg.feat_dtype == "bf16" else torch.float32,
                         track_edge_ids=track_edge_ids)


def make_pipeline(cfg: StreamConfig, graph, d_t: int = 100):
    """The config's DataPipeline: K most recent neighbours of src/dst/neg, a d_t
    cosine time encoding and, for the co-occurrence configs, per-position counts."""
    from tgengine_amd import DataPipeline, GatherSpec, NeighborSpec
    spec = GatherSpec(neighbors=NeighborSpec(k=cfg.k), co_occurrence=cfg.co_occurrence,
                      time_encoding=d_t)
    return DataPipeline(spec, graph)


def to_raw(cfg: StreamConfig, bt: dict, device="cuda"):
    """A generated batch as a RawBatch of device tensors (bf16 rows as bf16)."""
    import torch
    from tgengine_amd import RawBatch
    feat = torch.from_numpy(bt["feat"])
    if cfg.feat_dtype == "bf16":
        feat = feat.view(torch.bfloat16)
    return RawBatch(src=torch.from_numpy(bt["src"]).to(device),
                    dst=torch.from_numpy(bt["dst"]).to(device),
                    time=torch.from_numpy(bt["time"]).to(device),
                    edge_feat=feat.to(device),
                    neg=torch.from_numpy(bt["neg"]).to(device))
