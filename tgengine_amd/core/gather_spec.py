"""Gather specification, field-compatible with tgengine/core/gather_spec.py:6-32.

Extra fields (defaults keep the reference behaviour):

* ``time_encoding``: d_t of the fused FixedCosineTimeEncoder pass (0 = off).
  Frequencies w = 1/10**linspace(0, 9, d_t) in fp32 and bias 0
  (tgengine/nn/time_encoding.py:49-53) unless the pipeline is given an encoder.
* ``dt_mode``: "dygformer" (dt = f32(t_q) - f32(t), padding encodes to 0;
  tgengine/models/dygformer.py:273-279) or "tgn" (dt = f32(t_q - t), padding
  uses t = 0; tgengine/models/tgn.py:80).
* ``co_occurrence_mode``: "freq" (per-position counts over the K sequences,
  temporal_sample.cu:453-511) or "dygformer" (counts over the 1+K sequences with
  the node first, tgengine/models/dygformer.py:71-87).
* ``edge_ids``: also return the global event index of every neighbour.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class NeighborSpec:
    k: int = 32
    k2: int = 0
    strategy: str = "recency"
    include_edge_feat: bool = True
    for_nodes: tuple = ("src", "dst", "neg")

    @property
    def hops(self) -> int:
        return 2 if self.k2 > 0 else 1


@dataclass
class GatherSpec:
    neighbors: NeighborSpec = field(default_factory=NeighborSpec)
    co_occurrence: bool = False
    memory: bool = False
    time_encoding: int = 0
    dt_mode: str = "dygformer"
    co_occurrence_mode: str = "freq"
    edge_ids: bool = False
