"""Host-side logic that runs without a GPU: API compatibility with the reference
types, the work plans, the synthetic streams, the CPU-baseline restatement
against the oracle, the device cosine compiled for the host, and bench.py's
one-GPU guard."""
import dataclasses
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import spec as O
from oracle.refpath_torch import RefPathCPU
from tgengine_amd import (DataPipeline, GatherSpec, NeighborData, NeighborSpec, PreparedBatch,
                          RawBatch, TemporalGraph)
from tgengine_amd.pipeline import cosine_time_weights, event_plan
from tgengine_amd.synthetic import (CONFIGS, bf16_bits_to_f32, f32_to_bf16_bits, gen_batch,
                                    key_multiplier_ok, num_batches)

ROOT = Path(__file__).resolve().parent.parent


# ------------------------------------------------------------- API surface
def test_types_keep_reference_field_order():
    """Positional construction of the reference types keeps working (tgengine/core/batch.py)."""
    ref_nd = ["neighbor_ids", "timestamps", "edge_feats", "mask", "hop2_ids", "hop2_times",
              "hop2_feats", "hop2_mask"]
    assert [f.name for f in dataclasses.fields(NeighborData)][:len(ref_nd)] == ref_nd
    ref_rb = ["src", "dst", "time", "edge_feat", "neg", "neg_src", "edge_indices", "node_labels",
              "edge_labels", "node_feat"]
    assert [f.name for f in dataclasses.fields(RawBatch)] == ref_rb
    ref_pb = ["src", "dst", "neg", "time", "src_neighbors", "dst_neighbors", "neg_neighbors",
              "neg_src_neighbors", "neg_src", "co_occurrence", "memory_emb", "node_labels",
              "edge_labels", "node_feat"]
    assert [f.name for f in dataclasses.fields(PreparedBatch)][:len(ref_pb)] == ref_pb


def test_spec_defaults_match_reference():
    ns = NeighborSpec()
    assert (ns.k, ns.k2, ns.strategy, ns.include_edge_feat, ns.for_nodes) == \
        (32, 0, "recency", True, ("src", "dst", "neg"))
    assert ns.hops == 1 and NeighborSpec(k2=4).hops == 2
    gs = GatherSpec()
    assert (gs.co_occurrence, gs.memory, gs.time_encoding) == (False, False, 0)


def test_temporal_graph_has_no_cpu_path():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        TemporalGraph(10, edge_feat_dim=4, device="cpu")


def test_event_plan_layout():
    # [src(b), dst(b), neg(b*3 row-major), neg_src(b)] -> event p: p, b+p, 2b+3p+j, 5b+p
    b = 4
    plan = event_plan(b, [(0, 1), (b, 1), (2 * b, 3), (5 * b, 1)]).reshape(b, 6)
    for p in range(b):
        assert plan[p].tolist() == [p, b + p, 2 * b + 3 * p, 2 * b + 3 * p + 1, 2 * b + 3 * p + 2,
                                    5 * b + p]
    assert sorted(plan.reshape(-1).tolist()) == list(range(6 * b))


def test_cosine_weights_match_fixture():
    hexes = (ROOT / "tests" / "golden" / "time_weights_f32.txt").read_text().split()
    assert [f"{v:08x}" for v in cosine_time_weights(100).view(np.uint32)] == hexes


# ------------------------------------------------------------- synthetic streams
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_stream_batches_are_reproducible_and_well_formed(name):
    cfg = CONFIGS[name]
    a = gen_batch(cfg, 3)
    b = gen_batch(cfg, 3)
    for k in ("src", "dst", "time", "neg"):
        assert np.array_equal(a[k], b[k])
    assert np.array_equal(a["feat"].view(np.uint8), b["feat"].view(np.uint8))
    b0, b1 = gen_batch(cfg, 0, with_feats=False), gen_batch(cfg, 1, with_feats=False)
    for bt in (b0, b1, a):
        assert np.all(np.diff(bt["time"]) > 0)
        assert key_multiplier_ok(bt["time"], len(bt["src"]))
        lo, hi = cfg.src_range
        assert bt["src"].min() >= 0 and bt["src"].max() < cfg.num_nodes
        assert bt["dst"].min() >= 0 and bt["dst"].max() < cfg.num_nodes
    assert b0["time"][-1] < b1["time"][0]
    assert a["feat"].shape == (cfg.batch, cfg.feat_dim)
    assert a["neg"].shape == ((cfg.batch,) if cfg.n_neg == 1 else (cfg.batch, cfg.n_neg))


def test_stream_shapes_and_laws():
    c1 = CONFIGS["c1"]
    assert num_batches(c1) == 788
    bt = gen_batch(c1, 787)
    assert len(bt["src"]) == 157_474 - 787 * 200
    assert bt["src"].max() < 8227 and bt["dst"].min() >= 8227      # bipartite layout
    c3 = CONFIGS["c3"]
    bt = gen_batch(c3, 5, with_feats=False)
    _, counts = np.unique(np.concatenate([bt["src"], bt["dst"]]), return_counts=True)
    assert counts.max() > 1000                                      # Zipf(1.5) head
    assert gen_batch(CONFIGS["c4"], 0)["feat"].dtype == np.uint16   # bf16 bits


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32)
    x[:4] = [1.00390625, 1.01171875, -2.5e-39, 3.0e38]  # ties to even, denormal, large
    mine = f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, ref)
    assert np.array_equal(bf16_bits_to_f32(mine), torch.from_numpy(mine.view(np.int16)).view(
        torch.bfloat16).float().numpy())


# ------------------------------------------------------------- CPU baseline == oracle
@pytest.mark.parametrize("name,nb", [("c1", 12), ("c2", 12)])
def test_cpu_baseline_restatement_matches_oracle(name, nb):
    cfg = CONFIGS[name]
    cpu = RefPathCPU(cfg.num_nodes, cfg.feat_dim, cfg.buffer_size)
    ring = O.Ring.empty(cfg.num_nodes, cfg.buffer_size, cfg.feat_dim)
    w = O.time_weights(100)
    for i in range(nb):
        bt = gen_batch(cfg, i)
        src, dst, t = (torch.from_numpy(bt[k]) for k in ("src", "dst", "time"))
        neg = torch.from_numpy(bt["neg"])
        out = cpu.prepare(src, dst, neg, t, cfg.k, co=cfg.co_occurrence)
        nodes = np.concatenate([bt["src"], bt["dst"], bt["neg"].reshape(-1)])
        qt = np.concatenate([bt["time"]] * 3)
        o = O.recent(nodes, qt, cfg.k, None, ring if i else None, cfg.feat_dim)
        assert np.array_equal(out["ids"].numpy(), o.ids)
        assert np.array_equal(out["mask"].numpy(), o.mask)
        assert np.array_equal(out["times"].numpy(), o.times)
        assert np.array_equal(out["feats"].numpy(), o.feats)
        exact = O.time_encode_exact(O.dt_dygformer(qt, o.times), w, o.mask)
        assert np.max(np.abs(out["te"].numpy() - exact)) < 1e-6
        if cfg.co_occurrence:
            b = len(bt["src"])
            ea, ec = O.co_occurrence_freq(o.ids[:b], o.ids[b:2 * b])
            assert np.array_equal(out["co_a"].numpy(), ea) and np.array_equal(out["co_c"].numpy(), ec)
            assert np.array_equal(out["co_pair"].numpy(),
                                  O.co_pair_count(o.ids[:b], o.mask[:b], o.ids[b:2 * b], o.mask[b:2 * b]))
        cpu.advance(src, dst, t, torch.from_numpy(bt["feat"]))
        O.ring_advance(ring, bt["src"], bt["dst"], bt["time"], bt["feat"])
    assert np.array_equal(cpu.ids.numpy(), ring.ids) and np.array_equal(cpu.wp.numpy(), ring.wp)


# ------------------------------------------------------------- device cosine on the host
def _rev_frac_host(tmp_path, args):
    exe = tmp_path / "cos_check"
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-ffp-contract=off",
                        f"-I{ROOT / 'tgengine_amd' / 'csrc'}", str(ROOT / "tests" / "cos_check.cpp"),
                        "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], input=np.asarray(args, np.float32).tobytes(),
                         capture_output=True, check=True).stdout
    return np.frombuffer(out, np.float64)


def test_time_encoding_reduction_host_build(tmp_path):
    """rev_frac (the float64 half of the device cosine) against libm: cos(2 pi f) must
    equal cos(x) to 2e-7 below 2^29 (single rounding of x/(2 pi)) and to 1e-12 above,
    where the double-double table of frac(2^E/(2 pi)) does an exact reduction."""
    rng = np.random.default_rng(1)
    w = O.time_weights(100)
    dts = np.concatenate([10 ** rng.uniform(-3, 9, 4000), rng.uniform(-1e9, 1e9, 2000)]).astype(np.float32)
    small = O.time_args(dts, w).ravel()
    small = small[np.abs(small) < 2.0 ** 29]
    big = np.concatenate([
        (10 ** rng.uniform(np.log10(2.0 ** 29), 38.5, 20000)).astype(np.float32),
        -(10 ** rng.uniform(np.log10(2.0 ** 29), 38.5, 2000)).astype(np.float32),
        np.float32([2.0 ** 29, -(2.0 ** 29), 1e12, 3e38, -3e38, 1.0995116e12, 7.5e15,
                    np.finfo(np.float32).max]),
        (np.arange(1, 5000) * np.float32(2.0 ** 29 + 64)).astype(np.float32)])
    for args, tol in ((small, 2e-7), (big, 1e-12)):
        f = _rev_frac_host(tmp_path, args)
        assert np.all(np.abs(f) <= 0.5)
        err = np.abs(np.cos(2 * np.pi * f) - np.cos(args.astype(np.float64)))
        assert err.max() < tol, (tol, err.max(), args[err.argmax()])
    # closed forms: cos(0) = 1 (f = 0), and non-finite arguments give NaN
    f = _rev_frac_host(tmp_path, np.float32([0.0, -0.0, np.inf, -np.inf, np.nan]))
    assert f[0] == 0.0 and f[1] == 0.0 and np.all(np.isnan(f[2:]))


def test_time_encoding_reduction_table_is_generated():
    """tgx_rev_table.h is what gen_rev_table.py writes (pi from mpmath at 400 bits),
    and hi + lo equals frac(2^E / (2 pi)) in exact rational arithmetic for a few E."""
    from fractions import Fraction
    import importlib.util
    import mpmath
    src = ROOT / "tgengine_amd" / "csrc" / "gen_rev_table.py"
    spec = importlib.util.spec_from_file_location("gen_rev_table", src)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    rows = mod.table()
    text = (ROOT / "tgengine_amd" / "csrc" / "tgx_rev_table.h").read_text()
    for e, hi, lo in rows:
        assert f"{{{hi!r}, {lo!r}}}" in text and f"E = {e} " in text
    mpmath.mp.prec = 500
    pi = Fraction(int(mpmath.floor(mpmath.pi * mpmath.mpf(2) ** 480)), 2 ** 480)
    for e, hi, lo in rows[::17] + rows[-1:]:
        exact = Fraction(2 ** e) / (2 * pi)
        exact -= exact.numerator // exact.denominator
        assert abs(Fraction(hi) + Fraction(lo) - exact) < Fraction(1, 2 ** 100)


# ------------------------------------------------------------- bench contract
def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_byte_model():
    sys.path.insert(0, str(ROOT))
    import bench
    cfg = CONFIGS["c3"]
    # one query with V=5 valid rows: R = 16 + 32*12 + 5*16*2, W = 20*13 + 20*16*2 + 20*100*4
    assert bench.bytes_per_batch(cfg, 1, 5, 0) == 16 + 384 + 160 + 260 + 640 + 8000
    c2 = CONFIGS["c2"]
    assert bench.bytes_per_batch(c2, 3, 0, 1) - bench.bytes_per_batch(c2, 3, 0, 0) == 16 * c2.k
