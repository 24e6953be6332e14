"""Hot-path data types, field-compatible with tgengine/core/batch.py:10-100.

New optional outputs of the fused pass ride as extra fields with default None,
placed after the reference fields so positional construction keeps working:
``NeighborData.time_enc`` (Q,K,d_t) float32, ``NeighborData.edge_ids`` (Q,K)
int64 and ``PreparedBatch.co_occurrence_freq`` = (a_counts, c_counts) int32.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
from torch import Tensor


@dataclass
class NeighborData:
    """Result of a temporal neighbour query (reference batch.py:10-38).

    neighbor_ids (B,K) int32 (-1 = padding), timestamps (B,K) float64,
    edge_feats (B,K,d) in the graph's feature dtype, mask (B,K) bool;
    right-aligned, most recent last.
    """

    neighbor_ids: Tensor
    timestamps: Tensor
    edge_feats: Tensor
    mask: Tensor

    hop2_ids: Optional[Tensor] = None
    hop2_times: Optional[Tensor] = None
    hop2_feats: Optional[Tensor] = None
    hop2_mask: Optional[Tensor] = None

    time_enc: Optional[Tensor] = None   # (B, K, d_t) fused FixedCosineTimeEncoder output
    edge_ids: Optional[Tensor] = None   # (B, K) global event index, -1 = padding

    @property
    def batch_size(self) -> int:
        return self.neighbor_ids.shape[0]

    @property
    def seq_len(self) -> int:
        return self.neighbor_ids.shape[1]

    @property
    def device(self) -> torch.device:
        return self.neighbor_ids.device


@dataclass
class RawBatch:
    """A chronological batch of events before pipeline processing (batch.py:41-64)."""

    src: Tensor
    dst: Tensor
    time: Tensor
    edge_feat: Optional[Tensor] = None
    neg: Optional[Tensor] = None
    neg_src: Optional[Tensor] = None
    edge_indices: Optional[Tensor] = None

    node_labels: Optional[Tensor] = None
    edge_labels: Optional[Tensor] = None
    node_feat: Optional[Tensor] = None

    @property
    def batch_size(self) -> int:
        return self.src.shape[0]

    @property
    def device(self) -> torch.device:
        return self.src.device


@dataclass
class PreparedBatch:
    """Fully assembled model input (batch.py:67-100)."""

    src: Tensor
    dst: Tensor
    neg: Tensor
    time: Tensor

    src_neighbors: Optional[NeighborData]
    dst_neighbors: Optional[NeighborData]
    neg_neighbors: Optional[NeighborData]
    neg_src_neighbors: Optional[NeighborData] = None

    neg_src: Optional[Tensor] = None
    co_occurrence: Optional[Tensor] = None       # (B,) float32 shared-neighbour count
    memory_emb: Optional[Tensor] = None

    node_labels: Optional[Tensor] = None
    edge_labels: Optional[Tensor] = None
    node_feat: Optional[Tensor] = None

    # (src-side, dst-side) int32 per-position counts, see GatherSpec.co_occurrence_mode
    co_occurrence_freq: Optional[Tuple[Tensor, Tensor]] = None

    @property
    def batch_size(self) -> int:
        return self.src.shape[0]

    @property
    def device(self) -> torch.device:
        return self.src.device
