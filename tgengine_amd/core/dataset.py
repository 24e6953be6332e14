"""On-disk DyGLib datasets -> chronological RawBatch streams (reference
tgengine/core/dataset.py).

A DyGLib dataset directory ``<path>/<name>/`` holds ``ml_<name>.csv`` (columns
u, i, ts, one row per event), optionally ``ml_<name>.npy`` (edge features, one
row per event) and ``ml_<name>_node.npy`` (node features).  ``load_dataset``
reads them on the host, pads features to 172 columns, computes the
train/val/test split and the inductive-evaluation masks exactly as the
reference does (dataset.py:293-418), and ``TemporalDataset.get_batches``
(:123-182) hands out ``RawBatch``es.  On a GPU device a split is copied to HBM
once and every batch is a view of it, instead of one host-to-device copy per
batch and field.

Only the DyGLib family is read.  TGB / TGB-Seq directories (``tgbl-*``,
``tgbseq-*``) and downloading are not supported: there is no network, and
their negative-candidate files are pickles.
"""
from __future__ import annotations

import random
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import numpy as np
import torch
from torch import Tensor

from .batch import RawBatch

PAD_FEAT_DIM = 172
INDUCTIVE_SEED = 2020      # DyGLib's seed for the hidden test nodes (dataset.py:345)
INDUCTIVE_FRACTION = 0.1   # of all distinct nodes


@dataclass
class TemporalDataset:
    """A loaded temporal graph dataset, events ordered [train | val | test]
    (reference dataset.py:43-121); field names and meanings as there."""

    src: Tensor
    dst: Tensor
    time: Tensor
    edge_feat: Optional[Tensor]
    node_feat: Optional[Tensor]

    num_nodes: int
    num_edges: int

    train_end: int
    val_end: int

    new_node_val_mask: Optional[Tensor] = None
    new_node_test_mask: Optional[Tensor] = None
    inductive_edges: Optional[dict] = None

    val_neg_candidates: Optional[Tensor] = None
    test_neg_candidates: Optional[Tensor] = None

    node_labels: Optional[Tensor] = None
    edge_labels: Optional[Tensor] = None
    num_node_classes: Optional[int] = None
    num_edge_classes: Optional[int] = None

    split_strategy: str = "event"
    val_time: float = 0.0
    test_time: float = 0.0

    @property
    def edge_feat_dim(self) -> int:
        return self.edge_feat.shape[1] if self.edge_feat is not None else 0

    @property
    def node_feat_dim(self) -> int:
        return self.node_feat.shape[1] if self.node_feat is not None else 0

    @property
    def train_size(self) -> int:
        return self.train_end

    @property
    def val_size(self) -> int:
        return self.val_end - self.train_end

    @property
    def test_size(self) -> int:
        return self.num_edges - self.val_end

    def summary(self) -> str:
        """One line per split: event index range, size and time bounds."""
        out = [f"{self.num_nodes} nodes / {self.num_edges} events / edge features {self.edge_feat_dim}"
               f" / {self.split_strategy} split"]
        bounds = (("train", 0, self.train_end, f"time <= {self.val_time:.4g}"),
                  ("val", self.train_end, self.val_end,
                   f"{self.val_time:.4g} < time <= {self.test_time:.4g}"),
                  ("test", self.val_end, self.num_edges, f"time > {self.test_time:.4g}"))
        for name, lo, hi, cond in bounds:
            out.append(f"{name:>5} events [{lo}, {hi}) = {hi - lo}, {cond}")
        if self.inductive_edges is not None:
            n = len(self.inductive_edges["src"])
            out.append(f"{'new':>5} nodes withheld from training: {n} "
                       f"({n / max(self.num_nodes, 1):.1%} of all nodes)")
        return "\n".join(out)

    def split_range(self, split: str) -> tuple[int, int]:
        if split == "train":
            return 0, self.train_end
        if split == "val":
            return self.train_end, self.val_end
        if split == "test":
            return self.val_end, self.num_edges
        raise ValueError(f"Unknown split: {split}")

    def get_batches(self, split: str, batch_size: int, device: str = "cuda",
                    inductive_only: bool = False) -> list[RawBatch]:
        """Chronological batches of ``batch_size`` events of a split (reference
        :123-182); ``inductive_only`` keeps the val/test events that touch a node
        unseen in training.  The split's fields are moved to ``device`` once and
        the batches are row slices of them."""
        if batch_size <= 0:
            raise ValueError("batch_size must be positive")
        start, end = self.split_range(split)
        idx: Optional[Tensor] = None
        if inductive_only and split in ("val", "test"):
            mask = self.new_node_val_mask if split == "val" else self.new_node_test_mask
            if mask is not None:
                idx = torch.nonzero(mask[start:end]).reshape(-1) + start

        def take(t: Optional[Tensor]) -> Optional[Tensor]:
            if t is None:
                return None
            part = t[start:end] if idx is None else t.index_select(0, idx)
            return part.to(device)

        src = take(self.src)
        dst = take(self.dst)
        tim = take(self.time)
        feat = take(self.edge_feat)
        el = take(self.edge_labels)
        # node labels / node features are looked up by source node
        src_host = self.src[start:end] if idx is None else self.src.index_select(0, idx)
        nl = self.node_labels[src_host].to(device) if self.node_labels is not None else None
        nf = self.node_feat[src_host].to(device) if self.node_feat is not None else None

        n = src.shape[0]
        out = []
        for i in range(0, n, batch_size):
            j = min(i + batch_size, n)
            out.append(RawBatch(
                src=src[i:j], dst=dst[i:j], time=tim[i:j],
                edge_feat=feat[i:j] if feat is not None else None,
                node_labels=nl[i:j] if nl is not None else None,
                edge_labels=el[i:j] if el is not None else None,
                node_feat=nf[i:j] if nf is not None else None,
            ))
        return out


def compute_split_times(time_vals: np.ndarray, val_ratio: float, test_ratio: float,
                        strategy: str) -> tuple[float, float]:
    """(val_time, test_time) boundaries (reference dataset.py:185-211).

    "event": the linear-interpolation quantiles of the event times at
    1 - val - test and 1 - test (so 70% of events are train by default);
    "time": those fractions of the span [t_min, t_max].  The fractions are
    formed with the same floating-point operations as the reference so the
    boundaries agree bit for bit.
    """
    lo = 1 - val_ratio - test_ratio
    hi = 1 - test_ratio
    if strategy == "event":
        val_time, test_time = np.quantile(time_vals, [lo, hi])
    elif strategy == "time":
        t_min = float(time_vals.min())
        t_max = float(time_vals.max())
        span = t_max - t_min
        val_time = t_min + span * lo
        test_time = t_min + span * hi
    else:
        raise ValueError(f"split_strategy must be 'event' or 'time', got '{strategy}'")
    return float(val_time), float(test_time)


def _pad_features(a: np.ndarray) -> Tensor:
    """float32 rows, zero-padded on the right to PAD_FEAT_DIM columns (wider kept)."""
    if a.ndim != 2:
        raise ValueError(f"feature array must be 2-D, got shape {a.shape}")
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    if t.shape[1] < PAD_FEAT_DIM:
        t = torch.nn.functional.pad(t, (0, PAD_FEAT_DIM - t.shape[1]))
    return t


def _read_events(csv_path: Path) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    import pandas as pd
    df = pd.read_csv(str(csv_path))
    for c in ("u", "i", "ts"):
        if c not in df.columns:
            raise ValueError(f"{csv_path}: no column '{c}' (columns: {list(df.columns)})")
    return (df["u"].to_numpy(np.int64), df["i"].to_numpy(np.int64),
            df["ts"].to_numpy(np.float64))


def hidden_test_nodes(src: np.ndarray, dst: np.ndarray, time_vals: np.ndarray,
                      val_time: float) -> list:
    """The nodes hidden from training for inductive evaluation (reference
    dataset.py:344-351): INDUCTIVE_FRACTION of all distinct nodes, drawn without
    replacement by Python's ``random.sample`` seeded with INDUCTIVE_SEED, from
    the nodes of the events after val_time.  The candidates are enumerated as a
    Python set built by the same expression as the reference, since the draw
    depends on that enumeration order; a private generator leaves the global
    ``random`` state alone."""
    num_total_unique = len(set(src) | set(dst))
    later = time_vals > val_time
    test_node_set = set(src[later]) | set(dst[later])
    rng = random.Random(INDUCTIVE_SEED)
    return rng.sample(list(test_node_set), int(INDUCTIVE_FRACTION * num_total_unique))


def _print_split_summary(name: str, strategy: str, train_end: int, val_size: int, test_size: int,
                         val_time: float, test_time: float, num_nodes: int,
                         n_inductive: int) -> None:
    """Load-time report: dataset size, then the three split sizes and cut times."""
    total = train_end + val_size + test_size
    parts = [f"{name}: {total} events, {num_nodes} nodes, {strategy} split",
             f"train={train_end} val={val_size} test={test_size}",
             f"cuts at t={val_time:.4g} and t={test_time:.4g}"]
    if n_inductive > 0:
        parts.append(f"{n_inductive} new nodes withheld ({n_inductive / max(num_nodes, 1):.1%})")
    print("; ".join(parts))


def load_dyglib(dataset_name: str, base: Path, val_ratio: float = 0.15, test_ratio: float = 0.15,
                split_strategy: str = "event") -> TemporalDataset:
    """A DyGLib-format dataset with its splits and inductive masks (reference
    dataset.py:293-418).

    Events with time <= val_time are train, (val_time, test_time] val, the
    rest test.  Train events touching a hidden test node (hidden_test_nodes)
    are dropped from the train split and returned in ``inductive_edges``
    (file order).  An event of val/test is "new-node" when one of its ends
    never occurs in the kept train events.  Within a split, events keep the
    file's order.
    """
    base = Path(base)
    csv_path = base / f"ml_{dataset_name}.csv"
    if not csv_path.exists():
        raise FileNotFoundError(f"Dataset file not found: {csv_path}")
    src, dst, time_vals = _read_events(csv_path)
    if src.size == 0:
        raise ValueError(f"{csv_path}: no events")

    node_feat = None
    node_path = base / f"ml_{dataset_name}_node.npy"
    if node_path.exists():
        node_feat = _pad_features(np.load(str(node_path)))
    edge_feat = None
    feat_path = base / f"ml_{dataset_name}.npy"
    if feat_path.exists():
        edge_feat = _pad_features(np.load(str(feat_path)))
        if edge_feat.shape[0] < src.size:
            raise ValueError(f"{feat_path}: {edge_feat.shape[0]} rows for {src.size} events")

    num_nodes = int(max(src.max(), dst.max())) + 1

    val_time, test_time = compute_split_times(time_vals, val_ratio, test_ratio, split_strategy)
    train_mask = time_vals <= val_time
    val_mask = (time_vals > val_time) & (time_vals <= test_time)
    test_mask = time_vals > test_time

    hidden = np.asarray(hidden_test_nodes(src, dst, time_vals, val_time), dtype=np.int64)
    observed = ~(np.isin(src, hidden) | np.isin(dst, hidden))
    inductive_idx = np.flatnonzero(train_mask & ~observed)
    train_mask &= observed

    train_nodes = np.union1d(src[train_mask], dst[train_mask])
    new_nodes = np.setdiff1d(np.union1d(src, dst), train_nodes)
    touches_new = np.isin(src, new_nodes) | np.isin(dst, new_nodes)

    order = np.concatenate([np.flatnonzero(train_mask), np.flatnonzero(val_mask),
                            np.flatnonzero(test_mask)])
    inductive_edges = None
    if inductive_idx.size > 0:
        inductive_edges = {
            "src": torch.from_numpy(src[inductive_idx]),
            "dst": torch.from_numpy(dst[inductive_idx]),
            "time": torch.from_numpy(time_vals[inductive_idx]),
            "edge_feat": edge_feat[torch.from_numpy(inductive_idx)] if edge_feat is not None else None,
        }

    train_end = int(train_mask.sum())
    val_end = train_end + int(val_mask.sum())
    num_edges = val_end + int(test_mask.sum())
    order_t = torch.from_numpy(order)

    _print_split_summary(dataset_name, split_strategy, train_end, val_end - train_end,
                         num_edges - val_end, val_time, test_time,
                         int(np.union1d(src, dst).size), int(hidden.size))

    return TemporalDataset(
        src=torch.from_numpy(src[order]),
        dst=torch.from_numpy(dst[order]),
        time=torch.from_numpy(time_vals[order]),
        edge_feat=edge_feat[order_t] if edge_feat is not None else None,
        node_feat=node_feat,
        num_nodes=num_nodes,
        num_edges=num_edges,
        train_end=train_end,
        val_end=val_end,
        new_node_val_mask=torch.from_numpy((val_mask & touches_new)[order]),
        new_node_test_mask=torch.from_numpy((test_mask & touches_new)[order]),
        inductive_edges=inductive_edges,
        split_strategy=split_strategy,
        val_time=val_time,
        test_time=test_time,
    )


def load_dataset(dataset_name: str, dataset_path: str = "datasets", val_ratio: float = 0.15,
                 test_ratio: float = 0.15, split_strategy: str = "event",
                 auto_download: bool = False) -> TemporalDataset:
    """Load ``<dataset_path>/<dataset_name>`` (reference dataset.py:238-290);
    an underscore spelling of the directory is tried too.  DyGLib format only;
    nothing is downloaded."""
    if dataset_name.startswith(("tgbl-", "tgbseq-")):
        raise NotImplementedError(
            f"{dataset_name}: TGB / TGB-Seq datasets are not supported (DyGLib format only)")
    base = Path(dataset_path) / dataset_name
    if not base.exists():
        alt = Path(dataset_path) / dataset_name.replace("-", "_")
        if alt.exists():
            base = alt
    if not base.exists() and auto_download:
        raise FileNotFoundError(f"{base} not found and downloading is not supported")
    return load_dyglib(dataset_name, base, val_ratio, test_ratio, split_strategy)
