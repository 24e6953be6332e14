"""Streaming-loop parity of the HIP path against the CPU oracle on the five configs."""
import pytest

import stream_check

pytestmark = pytest.mark.gpu


def test_c1_stream_prefix():
    tot = stream_check.run("c1", 40, check=set(range(40)), ring_check_every=5)
    assert tot["checked"] == 40 and tot["valid"] > 0


def test_c2_stream_prefix_co_occurrence():
    tot = stream_check.run("c2", 40, check=set(range(0, 40, 2)), ring_check_every=5)
    assert tot["valid"] > 0


def test_c3_warm_window():
    tot = stream_check.run("c3", 120, check={1, 60, 119}, ring_check_every=40)
    assert tot["valid"] > 0


def test_c4_warm_window():
    tot = stream_check.run("c4", 40, check={1, 39}, ring_check_every=20)
    assert tot["valid"] > 0


def test_c5_warm_window():
    tot = stream_check.run("c5", 24, check={1, 23}, ring_check_every=12)
    assert tot["valid"] > 0


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_launch_matches_prepare(name):
    """DataPipeline.launch (the timing launch, no ring plan) gives prepare()'s
    outputs bit for bit: C2's 600 queries run the pair-plus-tiled-tail layout in
    both, C5's 24,576 keep every query of an event in its group."""
    import torch
    cfg = stream_check.CONFIGS[name]
    g = stream_check.make_graph(cfg)
    pipe = stream_check.make_pipeline(cfg, g)
    raws = [stream_check.to_raw(cfg, stream_check.gen_batch(cfg, i)) for i in range(8)]
    for i, raw in enumerate(raws):
        if i >= 4:
            out = pipe.launch(raw)
            pb = pipe.prepare(raw)
            groups = [pb.src_neighbors, pb.dst_neighbors, pb.neg_neighbors]
            for j, nb in enumerate(groups):
                for key, got in (("ids", nb.neighbor_ids), ("times", nb.timestamps),
                                 ("mask", nb.mask), ("te", nb.time_enc)):
                    assert torch.equal(out[key][j], got), (name, i, j, key)
                assert torch.equal(out["feats"][j].view(torch.uint8), nb.edge_feats.view(torch.uint8))
            assert torch.equal(out["co_a"], pb.co_occurrence_freq[0]), (name, i)
            assert torch.equal(out["co_c"], pb.co_occurrence_freq[1]), (name, i)
            assert torch.equal(out["co_pair"], pb.co_occurrence), (name, i)
        else:
            pipe.prepare(raw)
        g.advance(raw.src, raw.dst, raw.time, raw.edge_feat)
