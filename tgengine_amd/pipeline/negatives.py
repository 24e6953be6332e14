"""Negative sampling: the drop-in for tgengine/pipeline/negatives.py.

``HistoricalNegPool`` (reference :14-126) keeps, per source node, a pool of
``pool_size`` destination ids by reservoir sampling over every edge seen from
that node, on the device: ``update`` and ``sample`` are one libtgx call each
(tgx_negpool_update / tgx_negpool_sample).  Random numbers come from the
library's counter-based generator, seeded once per pool (from torch's global
generator unless ``seed`` is given) and advanced by one call counter, so a
pool replays identically for the same seed and calls.  With ``rng="torch"``
the draws come from torch's generator instead, in the reference's call order
and shapes (update: torch.rand(n) then torch.randint(0, pool_size, (n,));
sample: torch.rand(B), then torch.randint(0, num_nodes, (k,)) for the k
sources without history), so that for the same torch generator state the pool
and the samples are the reference's.  The reference's ``index_put_`` leaves a
slot two accepted edges of one batch pick to whichever write lands last; here
the later edge of the batch always takes it.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Optional

import torch
from torch import Tensor

from tgengine_amd.core import _lib
from tgengine_amd.core.temporal_graph import TemporalGraph, _stream_handle


class HistoricalNegPool:
    """For every source node, a fixed-size reservoir of the destinations it has
    linked to, so a negative can be drawn from that node's own history.

    Usage (as the reference):
        pool = HistoricalNegPool(num_nodes, pool_size=512, device="cuda")
        pool.update(src, dst)      # alongside graph.advance() for every batch
        neg = pool.sample(src)     # (B,) int64
    """

    PADDING: int = -1

    def __init__(self, num_nodes: int, pool_size: int = 512, device: str = "cuda",
                 seed: Optional[int] = None, rng: str = "counter"):
        if rng not in ("counter", "torch"):
            raise ValueError(f"rng must be 'counter' or 'torch', got {rng!r}")
        self.rng = rng
        self.num_nodes = int(num_nodes)
        self.pool_size = int(pool_size)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("HistoricalNegPool runs on the GPU only (libtgx)")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        _lib.lib()
        self._pool = torch.full((self.num_nodes, self.pool_size), self.PADDING, dtype=torch.int32,
                                device=self.device)
        self._count = torch.zeros(self.num_nodes, dtype=torch.int64, device=self.device)
        # the counter generator's seed (drawn from torch's generator unless given;
        # the torch mode draws nothing here, as the reference's constructor)
        self.seed = (int(seed) if seed is not None else
                     0 if rng == "torch" else int(torch.randint(0, 2 ** 62, (1,)).item()))
        self._call = 0
        self._status = torch.zeros(_lib.TGX_STATUS_WORDS, dtype=torch.int32, device=self.device)
        self._ws: Optional[Tensor] = None
        # the update's cell table (zero-filled once; every update leaves it zeroed)
        self._scratch = torch.zeros(int(_lib.lib().tgx_negpool_scratch_size()), dtype=torch.uint8,
                                    device=self.device)

    def _ids(self, t: Tensor) -> Tensor:
        return t.detach().to(self.device, torch.int64).contiguous().reshape(-1)

    def update(self, src: Tensor, dst: Tensor) -> None:
        """Add (src_i -> dst_i) edges by reservoir sampling (reference :45-103)."""
        n = int(src.shape[0])
        if n == 0:
            self._call += 1  # every update and sample call advances the counter
            return
        if dst.shape[0] != n:
            raise ValueError("src and dst must have the same length")
        s, d = self._ids(src), self._ids(dst)
        need = int(_lib.lib().tgx_negpool_update_workspace_size(n))
        if self._ws is None or self._ws.numel() < need:
            if self._ws is not None:
                # an update queued on another stream may still use the old one
                torch.cuda.synchronize(self.device)
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        if self.rng == "torch":
            # the reference's draws (negatives.py:78-86), by sorted position
            u_accept = torch.rand(n, device=self.device)
            slot_draw = torch.randint(0, self.pool_size, (n,), device=self.device)
            _lib.check(_lib.lib().tgx_negpool_update_draws(
                self._pool.data_ptr(), self._count.data_ptr(), self.num_nodes, self.pool_size,
                s.data_ptr(), d.data_ptr(), n, u_accept.data_ptr(), slot_draw.data_ptr(),
                self._ws.data_ptr(), self._ws.numel(), self._status.data_ptr(),
                _stream_handle(self.device)), "tgx_negpool_update_draws")
        else:
            _lib.check(_lib.lib().tgx_negpool_update(
                self._pool.data_ptr(), self._count.data_ptr(), self.num_nodes, self.pool_size,
                s.data_ptr(), d.data_ptr(), n, self.seed, self._call, self._ws.data_ptr(),
                self._ws.numel(), self._scratch.data_ptr(), self._scratch.numel(), self._status.data_ptr(),
                _stream_handle(self.device)), "tgx_negpool_update")
        self._call += 1

    def sample(self, src: Tensor) -> Tensor:
        """One historical negative per source, uniform over its pool; a random node
        for a source without history (reference :105-126)."""
        s = self._ids(src)
        out = torch.empty(s.shape[0], dtype=torch.int64, device=self.device)
        if self.rng == "torch":
            # the reference's draws (negatives.py:116-124): a uniform per query,
            # then a node per query without history, in query order
            u_slot = torch.rand(s.shape[0], device=self.device)
            if s.shape[0] > 0:
                _lib.check(_lib.lib().tgx_negpool_sample_draws(
                    self._pool.data_ptr(), self._count.data_ptr(), self.num_nodes, self.pool_size,
                    s.data_ptr(), s.shape[0], u_slot.data_ptr(), out.data_ptr(), self._status.data_ptr(),
                    _stream_handle(self.device)), "tgx_negpool_sample_draws")
                none = out < 0
                k = int(none.sum())
                if k:
                    out[none] = torch.randint(0, self.num_nodes, (k,), device=self.device)
            self._call += 1
            return out
        if s.shape[0] > 0:
            _lib.check(_lib.lib().tgx_negpool_sample(
                self._pool.data_ptr(), self._count.data_ptr(), self.num_nodes, self.pool_size,
                s.data_ptr(), s.shape[0], self.seed, self._call, out.data_ptr(),
                self._status.data_ptr(), _stream_handle(self.device)), "tgx_negpool_sample")
        self._call += 1
        return out


class NegativeStrategy(ABC):
    """Base class for negative sampling strategies (reference :129-151)."""

    @abstractmethod
    def sample(self, src: Tensor, dst: Tensor, time: Tensor, graph: TemporalGraph,
               edge_indices: Optional[Tensor] = None) -> Tensor:
        """(B,) or (B, N_neg) negative node ids."""

    def update(self, src: Tensor, dst: Tensor) -> None:
        """Take in a batch of edges, next to graph.advance(); strategies without
        state ignore it."""


class HistoricalNegative(NegativeStrategy):
    """Per-source historical negatives from a device pool (reference :174-192)."""

    def __init__(self, num_nodes: int, pool_size: int = 512, device: str = "cuda",
                 seed: Optional[int] = None, rng: str = "counter"):
        self._pool = HistoricalNegPool(num_nodes, pool_size=pool_size, device=device, seed=seed, rng=rng)
        self.num_nodes = num_nodes

    def update(self, src: Tensor, dst: Tensor) -> None:
        self._pool.update(src, dst)

    def sample(self, src: Tensor, dst: Tensor, time: Tensor, graph: TemporalGraph,
               edge_indices: Optional[Tensor] = None) -> Tensor:
        return self._pool.sample(src)


class FixedNegative(NegativeStrategy):
    """Fixed negative lists per global edge index (reference :212-229)."""

    def __init__(self, neg_lists: Tensor):
        self.neg_lists = neg_lists

    def sample(self, src: Tensor, dst: Tensor, time: Tensor, graph: TemporalGraph,
               edge_indices: Optional[Tensor] = None) -> Tensor:
        if edge_indices is None:
            raise ValueError("FixedNegative looks its lists up by global edge index: "
                             "pass the batch's edge_indices")
        return self.neg_lists[edge_indices.long()].to(src.device)
