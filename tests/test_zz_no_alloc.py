"""tgx_ring_append_static (the allocation-free ring update) against
tgx_ring_append, through the C ABI.

Two identical rings receive the same batches, one through each entry point:
a batch with hot nodes past the ring size and key collisions absent, then a
smaller batch (the static workspace keeps the first call's contents, which the
second must not depend on), then a batch with out-of-range node ids (the
diagnostics words).  Ring ids, times, feature rows, edge ids, write positions,
the per-node counters and the status words must be bit-identical after every
call.  A batch beyond the static workspace is refused with TGX_ERR_LIMIT.
"""
import ctypes

import numpy as np
import pytest
import torch

from tgengine_amd import TemporalGraph
from tgengine_amd.core import _lib

pytestmark = pytest.mark.gpu

N, B, D = 3000, 16, 12


def _graph():
    g = TemporalGraph(N, edge_feat_dim=D, buffer_size=B, device="cuda", track_edge_ids=True)
    g.freeze_csr()
    g._ensure_overflow()
    return g


def _batch(rng, b, bad=False):
    # a Zipf-like mix: a few hot nodes take most events, so rings overflow
    hot = rng.integers(0, 5, b)
    cold = rng.integers(0, N, b)
    src = np.where(rng.random(b) < 0.5, hot, cold).astype(np.int64)
    dst = rng.integers(0, N, b).astype(np.int64)
    if bad:
        src[::97] = N + 3
        dst[5::101] = -2
    t = np.sort(rng.uniform(4 * b, 8 * b, b))
    f = rng.standard_normal((b, D)).astype(np.float32)
    cu = lambda x: torch.from_numpy(x).cuda()  # noqa: E731
    return cu(src), cu(dst), cu(t), cu(f)


def _state(g):
    return {"ids": g._ov_ids.cpu().numpy(), "times": g._ov_times.cpu().numpy().view(np.int64),
            "feats": g._ov_feats.cpu().numpy().view(np.uint32), "eids": g._ov_eids.cpu().numpy(),
            "wp": g._ov_write_pos.cpu().numpy(), "scratch": g._ov_scratch[:N].cpu().numpy(),
            "status": g._status.cpu().numpy()}


def test_static_workspace_append_matches_workspace_append():
    L = _lib.lib()
    g1, g2 = _graph(), _graph()
    rng = np.random.default_rng(3)
    stream = torch.cuda.current_stream().cuda_stream
    eid = 0
    for b, bad in ((9000, False), (700, False), (2500, True)):
        src, dst, t, f = _batch(rng, b, bad)
        ws = torch.empty(int(L.tgx_ring_append_workspace_size(b)), dtype=torch.uint8, device="cuda")
        rc1 = L.tgx_ring_append(ctypes.byref(g1._ring()), src.data_ptr(), dst.data_ptr(), t.data_ptr(),
                                f.data_ptr(), b, eid, ws.data_ptr(), ws.numel(), g1._status.data_ptr(),
                                stream)
        _lib.check(rc1, "tgx_ring_append")
        rc2 = L.tgx_ring_append_static(ctypes.byref(g2._ring()), src.data_ptr(), dst.data_ptr(),
                                       t.data_ptr(), f.data_ptr(), b, eid, g2._status.data_ptr(), stream)
        _lib.check(rc2, "tgx_ring_append_static")
        eid += b
        s1, s2 = _state(g1), _state(g2)
        for k in s1:
            assert np.array_equal(s1[k], s2[k]), f"{k} differs after a batch of {b}"
        assert int(np.abs(s2["scratch"]).sum()) == 0  # per-node counters restored
    assert int(g2._status[_lib.TGX_ST_BAD_EVENT_NODE]) > 0
    assert int((g2._ov_write_pos > B).sum()) > 0  # hot rings overflowed
    # beyond the static workspace: refused before any device work
    big = 200_000
    assert L.tgx_ring_append_static(ctypes.byref(g2._ring()), src.data_ptr(), dst.data_ptr(),
                                    t.data_ptr(), None, big, 0, None, stream) == 3
    assert "static workspace" in L.tgx_last_error().decode()
