"""Writes dyglib_split.npz: a small synthetic DyGLib dataset and what the
reference's loader (tgengine/core/dataset.py:238-418, load_dataset ->
_load_dyglib) makes of it under both split strategies.

The hidden-test-node draw of that loader (Python ``random.sample`` over a
Python set, seed 2020) is fixed by nothing but the reference itself, so this
script imports the reference from /root/reference (read-only, never copied)
and records its outputs.  Run it in a container that has /root/reference:

    python tests/golden/make_dyglib_split.py

Inputs (the events, 4-column edge features with DyGLib's leading zero row,
3-column node features) are generated from a fixed seed and stored in the
fixture too, so tests/test_dataset.py rebuilds the same files.  Column 0 of an
edge-feature row is its row number, so the fixture keeps only the first four
output columns to identify rows.
"""
import sys
import tempfile
from pathlib import Path

import numpy as np

REFERENCE = "/root/reference"
NAME = "synth"


def make_inputs():
    """Sparse node ids (a Python set of them does not enumerate in sorted order)
    and events exactly at both boundaries of both strategies: with 1001 events
    the 0.70 / 0.85 quantiles are events 700 / 850, and with times spanning
    [0, 4000] the time-span boundaries are 2800 / 3400."""
    rng = np.random.default_rng(20260)
    E = 1001
    users = np.sort(rng.choice(np.arange(1, 6001), 120, replace=False))
    items = np.sort(rng.choice(np.arange(6001, 9001), 80, replace=False))
    u = users[rng.integers(0, users.size, E)]
    i = items[rng.integers(0, items.size, E)]
    u[:40] = users[rng.integers(0, 5, 40)]      # a few busy users early on
    ts = np.sort(rng.integers(1, 4000, E)).astype(np.float64)
    ts[0], ts[-1] = 0.0, 4000.0
    ts[700:720] = ts[700]                       # equal times at the event boundary
    for b in (2800.0, 3400.0):                  # and at the time-span boundaries
        k = int(np.searchsorted(ts, b))
        ts[k:k + 3] = b                         # those were >= b: still sorted
    ef = np.zeros((E + 1, 4), np.float32)       # row 0: DyGLib's padding row
    ef[1:, 1:] = rng.integers(-8, 8, (E, 3)) / np.float32(4)
    ef[:, 0] = np.arange(E + 1, dtype=np.float32)
    nf = (rng.integers(-8, 8, (9001, 3)) / 4).astype(np.float32)
    return u, i, ts, ef, nf


def write_files(base: Path, u, i, ts, ef, nf) -> None:
    import pandas as pd
    base.mkdir(parents=True, exist_ok=True)
    df = pd.DataFrame({"u": u, "i": i, "ts": ts, "label": np.zeros(len(u), np.int64),
                       "idx": np.arange(1, len(u) + 1)})
    df.to_csv(base / f"ml_{NAME}.csv")
    np.save(str(base / f"ml_{NAME}.npy"), ef)
    np.save(str(base / f"ml_{NAME}_node.npy"), nf)


def main() -> None:
    u, i, ts, ef, nf = make_inputs()
    sys.path.insert(0, REFERENCE)
    from tgengine.core.dataset import load_dataset  # noqa: E402  (the reference)

    out = {"u": u, "i": i, "ts": ts, "ef": ef, "nf": nf}
    with tempfile.TemporaryDirectory() as tmp:
        write_files(Path(tmp) / NAME, u, i, ts, ef, nf)
        for strategy in ("event", "time"):
            ds = load_dataset(NAME, tmp, split_strategy=strategy, auto_download=False)
            p = strategy + "_"
            out[p + "src"] = ds.src.numpy()
            out[p + "dst"] = ds.dst.numpy()
            out[p + "time"] = ds.time.numpy()
            out[p + "feat4"] = ds.edge_feat[:, :4].numpy()
            out[p + "feat_dim"] = np.int64(ds.edge_feat.shape[1])
            out[p + "feat_tail_zero"] = np.bool_(bool((ds.edge_feat[:, 4:] == 0).all()))
            out[p + "node_feat_is_input"] = np.bool_(
                np.array_equal(ds.node_feat[:, :3].numpy(), nf))
            out[p + "node_feat_dim"] = np.int64(ds.node_feat.shape[1])
            out[p + "node_tail_zero"] = np.bool_(bool((ds.node_feat[:, 3:] == 0).all()))
            out[p + "num_nodes"] = np.int64(ds.num_nodes)
            out[p + "ends"] = np.array([ds.train_end, ds.val_end, ds.num_edges], np.int64)
            out[p + "split_times"] = np.array([ds.val_time, ds.test_time], np.float64)
            out[p + "new_val"] = ds.new_node_val_mask.numpy()
            out[p + "new_test"] = ds.new_node_test_mask.numpy()
            ind = ds.inductive_edges
            out[p + "ind_src"] = ind["src"].numpy()
            out[p + "ind_dst"] = ind["dst"].numpy()
            out[p + "ind_time"] = ind["time"].numpy()
            out[p + "ind_feat4"] = ind["edge_feat"][:, :4].numpy()
    dest = Path(__file__).with_name("dyglib_split.npz")
    np.savez_compressed(dest, **out)
    print(f"wrote {dest}")


if __name__ == "__main__":
    main()
