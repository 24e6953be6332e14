"""The on-disk DyGLib loader (tgengine_amd/core/dataset.py) on the CPU.

Parity: tests/golden/dyglib_split.npz holds what the reference's loader
(tgengine/core/dataset.py:238-418) made of a synthetic dataset under both
split strategies, including the hidden-test-node draw, which nothing else
fixes.  Known answers and invariants cover the rest: quantile boundaries on a
dataset too small to hide any node, the time-span split, padding, batches.
"""
import random
from pathlib import Path

import numpy as np
import pandas as pd
import pytest
import torch

from tgengine_amd.core.dataset import (PAD_FEAT_DIM, TemporalDataset, compute_split_times,
                                       load_dataset)

GOLDEN = Path(__file__).parent / "golden" / "dyglib_split.npz"


def _write(base: Path, name: str, u, i, ts, ef=None, nf=None) -> None:
    base.mkdir(parents=True, exist_ok=True)
    pd.DataFrame({"u": u, "i": i, "ts": ts, "label": np.zeros(len(u), np.int64),
                  "idx": np.arange(1, len(u) + 1)}).to_csv(base / f"ml_{name}.csv")
    if ef is not None:
        np.save(str(base / f"ml_{name}.npy"), ef)
    if nf is not None:
        np.save(str(base / f"ml_{name}_node.npy"), nf)


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def synth_dir(golden, tmp_path_factory):
    root = tmp_path_factory.mktemp("dyglib")
    _write(root / "synth", "synth", golden["u"], golden["i"], golden["ts"], golden["ef"], golden["nf"])
    return root


@pytest.mark.parametrize("strategy", ["event", "time"])
def test_loader_matches_the_reference(golden, synth_dir, strategy):
    ds = load_dataset("synth", str(synth_dir), split_strategy=strategy)
    p = strategy + "_"
    assert [ds.train_end, ds.val_end, ds.num_edges] == golden[p + "ends"].tolist()
    assert [ds.val_time, ds.test_time] == golden[p + "split_times"].tolist()
    assert ds.num_nodes == int(golden[p + "num_nodes"])
    for field, key in (("src", "src"), ("dst", "dst"), ("time", "time")):
        got = getattr(ds, field)
        assert np.array_equal(got.numpy(), golden[p + key]), field
    assert ds.src.dtype == torch.int64 and ds.time.dtype == torch.float64
    assert ds.edge_feat.dtype == torch.float32
    assert ds.edge_feat.shape[1] == int(golden[p + "feat_dim"]) == PAD_FEAT_DIM
    assert np.array_equal(ds.edge_feat[:, :4].numpy(), golden[p + "feat4"])
    assert bool((ds.edge_feat[:, 4:] == 0).all()) == bool(golden[p + "feat_tail_zero"])
    assert ds.node_feat.shape[1] == int(golden[p + "node_feat_dim"])
    assert bool(golden[p + "node_feat_is_input"])
    assert np.array_equal(ds.node_feat[:, :3].numpy(), golden["nf"])
    assert bool((ds.node_feat[:, 3:] == 0).all()) == bool(golden[p + "node_tail_zero"])
    assert np.array_equal(ds.new_node_val_mask.numpy(), golden[p + "new_val"])
    assert np.array_equal(ds.new_node_test_mask.numpy(), golden[p + "new_test"])
    ind = ds.inductive_edges
    assert np.array_equal(ind["src"].numpy(), golden[p + "ind_src"])
    assert np.array_equal(ind["dst"].numpy(), golden[p + "ind_dst"])
    assert np.array_equal(ind["time"].numpy(), golden[p + "ind_time"])
    assert np.array_equal(ind["edge_feat"][:, :4].numpy(), golden[p + "ind_feat4"])


def test_loader_invariants(golden, synth_dir):
    """Splits partition the kept events by time; no train event touches a node
    of a new-node val/test event's hidden set; train + hidden edges are every
    event up to val_time."""
    ds = load_dataset("synth", str(synth_dir))
    t = ds.time.numpy()
    tr, va, te = t[:ds.train_end], t[ds.train_end:ds.val_end], t[ds.val_end:]
    assert (tr <= ds.val_time).all() and ((va > ds.val_time) & (va <= ds.test_time)).all()
    assert (te > ds.test_time).all()
    for part in (tr, va, te):  # file order kept, and the file is chronological
        assert (np.diff(part) >= 0).all()
    ts = golden["ts"]
    n_ind = ds.inductive_edges["src"].shape[0]
    assert ds.train_end + n_ind == int((ts <= ds.val_time).sum())
    assert ds.num_edges + n_ind == ts.size
    hidden = set(ds.inductive_edges["src"].tolist()) | set(ds.inductive_edges["dst"].tolist())
    train_nodes = set(ds.src[:ds.train_end].tolist()) | set(ds.dst[:ds.train_end].tolist())
    # every hidden event has at least one end outside the kept train nodes
    for s, d in zip(ds.inductive_edges["src"].tolist(), ds.inductive_edges["dst"].tolist()):
        assert s not in train_nodes or d not in train_nodes
    assert hidden
    new = ds.new_node_val_mask | ds.new_node_test_mask
    s, d = ds.src.numpy(), ds.dst.numpy()
    for j in range(ds.train_end, ds.num_edges):
        touches = s[j] not in train_nodes or d[j] not in train_nodes
        assert bool(new[j]) == touches
    assert not new[:ds.train_end].any()


def test_known_answer_small(tmp_path):
    """Ten events at t = 1..10 over five nodes: int(0.1 * 5) = 0 nodes hidden;
    quantiles 0.7 and 0.85 of 1..10 are 7.3 and 8.65 (linear interpolation)."""
    u = np.array([1, 2, 1, 3, 2, 1, 2, 4, 1, 5])
    i = np.array([2, 3, 3, 1, 1, 2, 3, 1, 5, 4])
    ts = np.arange(1, 11, dtype=np.float64)
    _write(tmp_path / "tiny", "tiny", u, i, ts, ef=np.ones((11, 2), np.float32))
    ds = load_dataset("tiny", str(tmp_path))
    assert ds.val_time == pytest.approx(7.3) and ds.test_time == pytest.approx(8.65)
    assert (ds.train_end, ds.val_end, ds.num_edges) == (7, 8, 10)
    assert ds.inductive_edges is None and ds.num_nodes == 6
    assert ds.src.tolist() == u.tolist() and ds.time.tolist() == ts.tolist()
    # nodes 4 and 5 never occur in train: events 8 (4->1), 9 (1->5), 10 (5->4)
    assert ds.new_node_val_mask.tolist() == [False] * 7 + [True, False, False]
    assert ds.new_node_test_mask.tolist() == [False] * 8 + [True, True]
    assert ds.edge_feat.shape == (10, PAD_FEAT_DIM)
    assert (ds.edge_feat[:, :2] == 1).all() and (ds.edge_feat[:, 2:] == 0).all()
    assert ds.node_feat is None and ds.node_feat_dim == 0
    assert "train events [0, 7) = 7" in ds.summary()

    dt = load_dataset("tiny", str(tmp_path), split_strategy="time")
    # span 9: boundaries 1 + 9 * 0.7 = 7.3 and 1 + 9 * 0.85 = 8.65, as "event" here
    assert (dt.train_end, dt.val_end) == (7, 8)


def test_split_times_closed_forms():
    t = np.array([0.0, 0.0, 0.0, 10.0, 100.0])
    # "event": quantile at 0.7 over 5 points sits 2.8 of the way: between 0 and 10
    v, w = compute_split_times(t, 0.15, 0.15, "event")
    assert v == pytest.approx(8.0) and w == pytest.approx(46.0)
    v, w = compute_split_times(t, 0.15, 0.15, "time")
    assert v == pytest.approx(70.0) and w == pytest.approx(85.0)
    v, w = compute_split_times(t, 0.1, 0.2, "time")
    assert v == pytest.approx(70.0) and w == pytest.approx(80.0)
    with pytest.raises(ValueError):
        compute_split_times(t, 0.15, 0.15, "random")


def test_get_batches(synth_dir):
    ds = load_dataset("synth", str(synth_dir))
    for split, (a, b) in (("train", (0, ds.train_end)), ("val", (ds.train_end, ds.val_end)),
                          ("test", (ds.val_end, ds.num_edges))):
        batches = ds.get_batches(split, 100, device="cpu")
        assert [x.batch_size for x in batches[:-1]] == [100] * (len(batches) - 1)
        assert torch.equal(torch.cat([x.src for x in batches]), ds.src[a:b])
        assert torch.equal(torch.cat([x.time for x in batches]), ds.time[a:b])
        assert torch.equal(torch.cat([x.edge_feat for x in batches]), ds.edge_feat[a:b])
        assert torch.equal(torch.cat([x.node_feat for x in batches]), ds.node_feat[ds.src[a:b]])
        assert all(x.neg is None and x.edge_labels is None for x in batches)
    for split, mask in (("val", ds.new_node_val_mask), ("test", ds.new_node_test_mask)):
        batches = ds.get_batches(split, 7, device="cpu", inductive_only=True)
        idx = torch.nonzero(mask).reshape(-1)
        assert len(idx) > 0
        assert torch.equal(torch.cat([x.dst for x in batches]), ds.dst[idx])
        assert torch.equal(torch.cat([x.edge_feat for x in batches]), ds.edge_feat[idx])
    # inductive_only has no meaning for train
    assert len(ds.get_batches("train", 10 ** 6, device="cpu", inductive_only=True)) == 1
    with pytest.raises(ValueError):
        ds.get_batches("dev", 10, device="cpu")
    with pytest.raises(ValueError):
        ds.get_batches("train", 0, device="cpu")


def test_load_dataset_paths_and_errors(tmp_path, golden):
    _write(tmp_path / "my_set", "my-set", golden["u"][:50], golden["i"][:50], golden["ts"][:50])
    ds = load_dataset("my-set", str(tmp_path))  # the underscore spelling of the directory
    assert ds.edge_feat is None and ds.edge_feat_dim == 0
    assert isinstance(ds, TemporalDataset)
    with pytest.raises(FileNotFoundError):
        load_dataset("absent", str(tmp_path))
    with pytest.raises(FileNotFoundError):
        load_dataset("absent", str(tmp_path), auto_download=True)
    with pytest.raises(NotImplementedError):
        load_dataset("tgbl-wiki", str(tmp_path))
    _write(tmp_path / "short", "short", golden["u"][:50], golden["i"][:50], golden["ts"][:50],
           ef=np.zeros((20, 3), np.float32))
    with pytest.raises(ValueError):
        load_dataset("short", str(tmp_path))


def test_global_random_state_untouched(synth_dir):
    random.seed(99)
    before = random.random()
    random.seed(99)
    load_dataset("synth", str(synth_dir))
    assert random.random() == before
