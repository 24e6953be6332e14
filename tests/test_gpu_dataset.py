"""A DyGLib dataset from disk through the device path, as the reference's
Engine drives it (engine/__init__.py:168-195, :602-608): load, replay the train
split into the graph, freeze the CSR, then per val batch sample historical
negatives, prepare (CSR window merged with the ring, 172-column features, time
encodings, co-occurrence) and advance.  Every prepared batch is compared with
the oracle on the same CSR and ring state."""
import types

import numpy as np
import pytest
import torch

import stream_check
from oracle import spec as O
from test_dataset import GOLDEN, _write
from tgengine_amd import DataPipeline, GatherSpec, NeighborSpec, TemporalGraph
from tgengine_amd.core.dataset import PAD_FEAT_DIM, load_dataset
from tgengine_amd.pipeline.negatives import HistoricalNegPool

pytestmark = pytest.mark.gpu


def test_dyglib_split_through_the_pipeline(tmp_path):
    with np.load(GOLDEN) as z:
        u, i, ts, ef, nf = z["u"], z["i"], z["ts"], z["ef"], z["nf"]
    _write(tmp_path / "synth", "synth", u, i, ts, ef, nf)
    ds = load_dataset("synth", str(tmp_path))
    N, d, K, ring_size = ds.num_nodes, PAD_FEAT_DIM, 16, 8
    print(f"dataset: {ds.num_edges} events, {N} nodes; K={K}", flush=True)

    g = TemporalGraph(N, edge_feat_dim=d, device="cuda", buffer_size=ring_size)
    pool = HistoricalNegPool(N, pool_size=8, device="cuda", seed=11)
    events, base = [], 0
    for rb in ds.get_batches("train", 200, device="cuda"):
        g.advance(rb.src, rb.dst, rb.time, rb.edge_feat)
        pool.update(rb.src, rb.dst)
        events.append((rb.src.cpu().numpy(), rb.dst.cpu().numpy(), rb.time.cpu().numpy(),
                       rb.edge_feat.cpu().numpy(), base))
        base += rb.batch_size
    g.freeze_csr()
    csr = O.csr_freeze(N, d, events)
    ring = O.Ring.empty(N, ring_size, d, np.float32)

    cfg = types.SimpleNamespace(k=K, feat_dim=d, feat_dtype="f32", co_occurrence=True)
    pipe = DataPipeline(GatherSpec(neighbors=NeighborSpec(k=K), co_occurrence=True,
                                   time_encoding=100), g)
    w = O.time_weights(100)
    valid = 0
    for j, rb in enumerate(ds.get_batches("val", 50, device="cuda")):
        rb.neg = pool.sample(rb.src)
        pb = pipe.prepare(rb)
        bt = {"src": rb.src.cpu().numpy(), "dst": rb.dst.cpu().numpy(),
              "time": rb.time.cpu().numpy(), "neg": rb.neg.cpu().numpy()}
        assert not O.key_collision(bt["time"], len(bt["src"]))
        st = stream_check.compare_prepared(cfg, pb, bt, ring, w, f"val batch {j}", csr=csr)
        valid += st["valid"]
        g.advance(rb.src, rb.dst, rb.time, rb.edge_feat)
        pool.update(rb.src, rb.dst)
        O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], rb.edge_feat.cpu().numpy())
    assert valid > 0
    s = g.status()
    assert not (s["bad_event_nodes"] or s["key_collisions"] or s["bad_query_nodes"]), s
