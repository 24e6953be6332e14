"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/tgx.h declares, its struct layouts match the ctypes mirror, and every
argument check returns the documented error before anything is launched."""
import ctypes
import re
import subprocess
import threading
from pathlib import Path

import pytest

from tgengine_amd.core import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tgx.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tgx_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 7
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert L.tgx_abi_version() == _lib.TGX_ABI_VERSION == 17
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True).stdout
    exported = set(re.findall(r"\bT (tgx_\w+)", nm))
    assert set(names) <= exported


LAYOUT_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "tgx.h"
#define F(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
#define S(T) printf(#T " %zu\n", sizeof(T));
int main(void) {
  S(tgx_ring) F(tgx_ring, num_nodes) F(tgx_ring, slots) F(tgx_ring, ids) F(tgx_ring, eids)
  F(tgx_ring, scratch)
  S(tgx_csr) F(tgx_csr, offsets) F(tgx_csr, eids) F(tgx_csr, max_time)
  S(tgx_query_group) F(tgx_query_group, count) F(tgx_query_group, times_per)
  F(tgx_query_group, flags) F(tgx_query_group, valid)
  S(tgx_recent_args) F(tgx_recent_args, k) F(tgx_recent_args, plan) F(tgx_recent_args, group)
  F(tgx_recent_args, plan_mode) F(tgx_recent_args, num_groups) F(tgx_recent_args, out_eids) F(tgx_recent_args, d_t)
  F(tgx_recent_args, te_w) F(tgx_recent_args, dt_mode) F(tgx_recent_args, out_te)
  F(tgx_recent_args, co_mode) F(tgx_recent_args, co_a) F(tgx_recent_args, status)
  F(tgx_recent_args, num_query_groups) F(tgx_recent_args, query_groups)
  F(tgx_recent_args, timing_start) F(tgx_recent_args, timing_stop)
  F(tgx_recent_args, append_src) F(tgx_recent_args, append_b) F(tgx_recent_args, append_workspace_bytes)
  F(tgx_recent_args, event_query_groups)
  F(tgx_recent_args, te_bound_w)
  F(tgx_recent_args, te_bound_b)
  S(tgx_csr_build_args) F(tgx_csr_build_args, num_entries) F(tgx_csr_build_args, event)
  F(tgx_csr_build_args, num_events) F(tgx_csr_build_args, feat_dtype) F(tgx_csr_build_args, out_offsets)
  F(tgx_csr_build_args, out_eids) F(tgx_csr_build_args, workspace_bytes) F(tgx_csr_build_args, status)
  F(tgx_csr_build_args, flags) F(tgx_csr_build_args, call_starts) F(tgx_csr_build_args, num_calls)
  return 0;
}
"""


def test_struct_layouts_match_ctypes(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(LAYOUT_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    mirror = {"tgx_ring": _lib.TgxRing, "tgx_csr": _lib.TgxCsr,
              "tgx_query_group": _lib.TgxQueryGroup, "tgx_recent_args": _lib.TgxRecentArgs,
              "tgx_csr_build_args": _lib.TgxCsrBuildArgs}
    for line in out.splitlines():
        key, val = line.split()
        if "." in key:
            t, f = key.split(".")
            assert getattr(mirror[t], f).offset == int(val), key
        else:
            assert ctypes.sizeof(mirror[key]) == int(val), key


def _err():
    return _lib.lib().tgx_last_error().decode()


def test_recent_argument_checks():
    L = _lib.lib()
    assert L.tgx_recent(None, None, None, None) == 1 and "args is NULL" in _err()
    a = _lib.TgxRecentArgs(k=0, group=1, num_queries=1, num_groups=1)
    assert L.tgx_recent(None, None, ctypes.byref(a), None) == 3 and "k=0" in _err()
    a = _lib.TgxRecentArgs(k=4, group=9, num_queries=1, num_groups=1)
    assert L.tgx_recent(None, None, ctypes.byref(a), None) == 3 and "group=9" in _err()
    a = _lib.TgxRecentArgs(k=4, group=1, num_queries=0, num_groups=0)
    assert L.tgx_recent(None, None, ctypes.byref(a), None) == 0  # nothing to do
    a = _lib.TgxRecentArgs(k=4, group=1, num_queries=5, num_groups=5)
    assert L.tgx_recent(None, None, ctypes.byref(a), None) == 1 and "must not be NULL" in _err()
    a = _lib.TgxRecentArgs(k=4, group=1, num_queries=5, num_groups=5, num_query_groups=5)
    assert L.tgx_recent(None, None, ctypes.byref(a), None) == 3 and "query groups" in _err()
    # no ring and no CSR: nothing sizes the feature rows
    a = _lib.TgxRecentArgs(k=4, group=1, num_queries=5, num_groups=5, nodes=8, times=8,
                           out_ids=8, out_times=8, out_mask=8, out_feats=8)
    assert L.tgx_recent(None, None, ctypes.byref(a), None) == 1 and "out_feats" in _err()
    ring = _lib.TgxRing(num_nodes=10, slots=65, feat_dim=2, feat_dtype=0, ids=8, times=8)
    a = _lib.TgxRecentArgs(k=4, group=1, num_queries=5, num_groups=5, nodes=8, times=8,
                           out_ids=8, out_times=8, out_mask=8)
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 3 and "slots=65" in _err()
    ring.slots = 4
    ring.feat_dtype = 7
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 2
    ring.feat_dtype = 0
    a.d_t = 600
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 3 and "d_t=600" in _err()
    a.d_t = 10
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "te_w" in _err()
    a.d_t = 0
    a.co_mode = 1
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "group >= 2" in _err()
    a.co_mode = 0
    a.dt_mode = 5
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "dt_mode" in _err()
    a.dt_mode = 0
    a.timing_start = 8
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "timing" in _err()
    a.timing_start = 0
    a.plan_mode = 7
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "plan_mode" in _err()
    a.plan_mode = _lib.TGX_PLAN_LIST  # a list plan needs its array
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "plan array" in _err()
    a.plan_mode = _lib.TGX_PLAN_TILES


def _shape(ring, csr, a):
    out = (ctypes.c_int64 * 8)()
    rc = _lib.lib().tgx_recent_launch_shape(ring, csr, ctypes.byref(a), out)
    return rc, list(out)


def test_co_occurrence_needs_a_plan_group():
    """Co-occurrence pairs queries 0 and 1 of a plan group, so a tiled launch
    (no plan array, no event-major plan) is refused instead of pairing queries
    of the wrong workgroups and leaving output rows unwritten."""
    L = _lib.lib()
    ring = _lib.TgxRing(num_nodes=10, slots=4, feat_dim=2, feat_dtype=0, ids=8, times=8)
    a = _lib.TgxRecentArgs(k=4, group=2, num_queries=6, num_groups=3, nodes=8, times=8,
                           out_ids=8, out_times=8, out_mask=8, co_mode=_lib.TGX_CO_FREQ, co_a=8, co_c=8)
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1
    assert "TGX_PLAN_EVENTS" in _err()
    # event-major groups need query groups whose per-event counts sum to `group`
    a.plan_mode = _lib.TGX_PLAN_EVENTS
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "event-major" in _err()
    a.num_query_groups = 2
    for g in range(2):
        a.query_groups[g].nodes = 8
        a.query_groups[g].times = 8
        a.query_groups[g].count = 3
        a.query_groups[g].times_per = 1
    rc, sh = _shape(ctypes.byref(ring), None, a)
    assert rc == 0, _err()
    assert sh[0] == 3 and sh[5] == 2 and sh[1] == 64 * 2 * sh[4]  # one event (2 queries) per workgroup
    a.query_groups[1].count = 2  # not one query per event
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "times_per" in _err()


def test_launch_shapes_stay_within_the_kernel_bounds():
    """Every tiled launch fits the kernel's 512-thread bound and the LDS, for
    every query count on both sides of the split rule, K and group: a tiny
    batch (one query, K=3, no ring) once asked for four query slots of eight
    split wavefronts, a 2048-thread block that the runtime refused."""
    csr = _lib.TgxCsr(num_nodes=10, num_entries=5, feat_dim=4, feat_dtype=0, offsets=8, ids=8,
                      times=8, feats=8)
    ring = _lib.TgxRing(num_nodes=10, slots=32, feat_dim=4, feat_dtype=0, ids=8, times=8, feats=16)
    ring64 = _lib.TgxRing(num_nodes=10, slots=64, feat_dim=4, feat_dtype=0, ids=8, times=8, feats=16)
    for Q in (1, 2, 3, 511, 512, 513, 1024, 2049, 4096, 4097, 8192, 8193, 20000):
        for k in (1, 3, 20, 64, 256, 300, 512):
            for group in (1, 2, 4, 8):
                for store in ((None, ctypes.byref(csr)), (ctypes.byref(ring), None),
                              (ctypes.byref(ring64), ctypes.byref(csr))):
                    a = _lib.TgxRecentArgs(k=k, group=group, num_queries=Q, nodes=8, times=8,
                                           out_ids=8, out_times=8, out_mask=8, out_feats=16)
                    rc, sh = _shape(store[0], store[1], a)
                    assert rc == 0, _err()
                    blocks, threads, lds, m, split, qpb = sh[:6]
                    assert 64 <= threads <= 512 and threads % 64 == 0
                    assert lds <= 160 * 1024
                    assert threads // 64 == (qpb // m) * split
                    assert blocks * qpb >= Q  # every query has a slot
                    assert qpb // m <= group
    a = _lib.TgxRecentArgs(k=3, group=4, num_queries=1, nodes=8, times=8, out_ids=8, out_times=8,
                           out_mask=8, out_feats=16)
    rc, sh = _shape(None, ctypes.byref(csr), a)
    # one query over 8 waves: without a ring, two workgroups of 4
    assert rc == 0 and sh[1] == 256 and sh[4] == 4 and sh[0] == 2 and sh[5] == 1
    rc, sh = _shape(ctypes.byref(ring), ctypes.byref(csr), a)
    assert rc == 0 and sh[1] == 512 and sh[4] == 8 and sh[0] == 1  # with a ring: one workgroup


def test_ring_less_launches_pack_queries_in_csr_window():
    """A CSR-only tiled launch of more than 2,048 queries at K <= 64 with rows of at
    most 64 bytes runs csr_window: 64 / Bp queries per wavefront (Bp = the power of
    two >= max(K, 16)), `group` wavefronts per workgroup, no split; a larger K,
    wider rows or a small launch take recent_fused's ring-less copy, one query per
    wavefront."""
    csr = _lib.TgxCsr(num_nodes=10, num_entries=5, feat_dim=8, feat_dtype=_lib.TGX_BF16, offsets=8,
                      ids=8, times=8, feats=16)
    for k, m in ((1, 4), (16, 4), (17, 2), (20, 2), (32, 2), (33, 1), (64, 1)):
        a = _lib.TgxRecentArgs(k=k, group=4, num_queries=12000, nodes=8, times=8, out_ids=8,
                               out_times=8, out_mask=8, out_feats=16)
        rc, sh = _shape(None, ctypes.byref(csr), a)
        assert rc == 0, _err()
        assert sh[3] == m and sh[4] == 1 and sh[1] == 256
        assert sh[0] == -(-12000 // (4 * m))
        if m > 1:  # few queries: one per wave, split
            a.num_queries = 2000
            assert _shape(None, ctypes.byref(csr), a)[1][3] == 1
    a = _lib.TgxRecentArgs(k=65, group=4, num_queries=12000, nodes=8, times=8, out_ids=8,
                           out_times=8, out_mask=8, out_feats=16)
    assert _shape(None, ctypes.byref(csr), a)[1][3] == 1
    wide = _lib.TgxCsr(num_nodes=10, num_entries=5, feat_dim=40, feat_dtype=_lib.TGX_BF16, offsets=8,
                       ids=8, times=8, feats=16)  # 80-byte rows
    a.k = 20
    assert _shape(None, ctypes.byref(wide), a)[1][3] == 1


def test_fastdiv_range_is_checked():
    """Feature chunks are divided by the row's chunk count with a multiply-high
    that is exact for dividends below 2^32 / chunks: wider rows are refused."""
    ring = _lib.TgxRing(num_nodes=10, slots=4, feat_dim=30001, feat_dtype=_lib.TGX_BF16, ids=8,
                        times=8, feats=2)
    a = _lib.TgxRecentArgs(k=32, group=1, num_queries=5, nodes=8, times=8, out_ids=8, out_times=8,
                           out_mask=8, out_feats=2)
    assert _lib.lib().tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 3
    assert "index range" in _err()
    a.k = 4  # 4 * 30001^2 < 2^32
    assert _shape(ctypes.byref(ring), None, a)[0] == 0


def test_ring_append_argument_checks():
    L = _lib.lib()
    ws = ctypes.create_string_buffer(1 << 16)
    assert L.tgx_ring_append(None, 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 1
    ring = _lib.TgxRing(num_nodes=10, slots=4, feat_dim=2, feat_dtype=0, ids=8, times=8, feats=8,
                        write_pos=8, scratch=8)
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, -1, 0, ws, 1 << 16, None, None) == 1
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, 0, 0, None, 0, None, None) == 0
    ring.scratch = 0
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 1
    assert "scratch" in _err()
    ring.scratch = 8
    ring.slots = 65
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 3
    ring.slots = 4
    ring.feat_dtype = 3
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 2
    ring.feat_dtype = 0
    need = L.tgx_ring_append_workspace_size(4)
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, 4, 0, ws, need - 1, None, None) == 1
    assert "workspace" in _err()
    ring.num_nodes = 1 << 31
    assert L.tgx_ring_append(ctypes.byref(ring), 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 3


def test_ring_plan_commit_discard_argument_checks():
    L = _lib.lib()
    ws = ctypes.create_string_buffer(1 << 16)
    ring = _lib.TgxRing(num_nodes=10, slots=4, feat_dim=2, feat_dtype=0, ids=8, times=8, feats=8,
                        write_pos=8, scratch=8)
    r = ctypes.byref(ring)
    assert L.tgx_ring_plan(None, 8, 8, 8, 4, ws, 1 << 16, None) == 1
    assert L.tgx_ring_commit(None, 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 1
    assert L.tgx_ring_discard(None, 8, 8, 4, ws, 1 << 16, None) == 1
    # empty batches are no-ops for every half
    assert L.tgx_ring_plan(r, 8, 8, 8, 0, None, 0, None) == 0
    assert L.tgx_ring_commit(r, 8, 8, 8, None, 0, 0, None, 0, None, None) == 0
    assert L.tgx_ring_discard(r, 8, 8, 0, None, 0, None) == 0
    # the plan needs times, the discard does not
    assert L.tgx_ring_plan(r, 8, 8, None, 4, ws, 1 << 16, None) == 1
    assert "tgx_ring_plan" in _err()
    need = L.tgx_ring_append_workspace_size(4)
    assert L.tgx_ring_discard(r, 8, 8, 4, ws, need - 1, None) == 1
    assert "workspace" in _err()
    ring.slots = 65
    assert L.tgx_ring_commit(r, 8, 8, 8, None, 4, 0, ws, 1 << 16, None, None) == 3
    ring.slots = 4
    # the workspace is read as 16-byte vectors
    base = ctypes.addressof(ws)
    odd = base + (-base) % 16 + 4
    assert L.tgx_ring_plan(r, 8, 8, 8, 4, odd, (1 << 16) - 64, None) == 1
    assert "aligned" in _err()


def test_static_append_limits():
    """tgx_ring_append_static refuses batches beyond its static workspace before
    touching the device, and an empty batch is a no-op."""
    L = _lib.lib()
    cap = L.tgx_ring_append_static_max_bytes()
    assert cap == 2 << 20
    ring = _lib.TgxRing(num_nodes=10, slots=4, feat_dim=2, feat_dtype=0, ids=8, times=8, feats=8,
                        write_pos=8, scratch=8)
    big = 1
    while L.tgx_ring_append_workspace_size(big) <= cap:
        big *= 2
    assert big > 100_000  # about 100,000 events fit
    assert L.tgx_ring_append_static(ctypes.byref(ring), 8, 8, 8, None, big, 0, None, None) == 3
    assert "static workspace" in _err()
    assert L.tgx_ring_append_static(ctypes.byref(ring), 8, 8, 8, None, -1, 0, None, None) == 1
    assert L.tgx_ring_append_static(ctypes.byref(ring), 8, 8, 8, None, 0, 0, None, None) == 0
    assert L.tgx_ring_append_static(None, 8, 8, 8, None, 0, 0, None, None) == 1


def test_size_queries():
    L = _lib.lib()
    # per-node counter + 8-entry node list, and 32 control words (16-byte aligned)
    assert L.tgx_ring_scratch_size(1000) == (9 * 1000 + 32) * 4
    assert L.tgx_ring_scratch_size(1001) == (9 * 1001 + 3 + 32) * 4
    n = 2 * 4000
    ws = L.tgx_ring_append_workspace_size(4000)
    # tickets (or entry nodes), four-launch lists, groups, large groups
    assert ws >= 4 * n + 4 * n + 4 * (n // 2 + 1) + 4 * (n // 9 + 1)
    assert L.tgx_ring_append_workspace_size(0) > 0


def test_csr_build_argument_checks():
    L = _lib.lib()
    a = _lib.TgxCsrBuildArgs(num_nodes=0, num_entries=0)
    assert L.tgx_csr_build(ctypes.byref(a), None) == 3 and "num_nodes" in _err()
    a = _lib.TgxCsrBuildArgs(num_nodes=10, num_entries=-1)
    assert L.tgx_csr_build(ctypes.byref(a), None) == 3
    a = _lib.TgxCsrBuildArgs(num_nodes=10, num_entries=5, out_offsets=8)
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "must not be NULL" in _err()
    a = _lib.TgxCsrBuildArgs(num_nodes=10, num_entries=5, out_offsets=8, from_=8, to=8, time=8,
                             out_ids=8, out_times=8, feat_dim=4, feat_dtype=_lib.TGX_F32)
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "out_feats" in _err()
    a.out_feats = 8
    a.feats = 8
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "event" in _err()
    a.event = 8
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "workspace" in _err()
    a.feat_dtype = 9
    assert L.tgx_csr_build(ctypes.byref(a), None) == 2
    assert L.tgx_csr_build(None, None) == 1
    # build modes: pairs and by-call exclude each other, runs need by-call, by-call
    # needs its call starts, and every mode takes events (an even entry count)
    a = _lib.TgxCsrBuildArgs(num_nodes=10, num_entries=6, out_offsets=8, from_=8, to=8, time=8,
                             out_ids=8, out_times=8, flags=_lib.TGX_CSR_EVENT_PAIRS | _lib.TGX_CSR_EVENTS_BY_CALL)
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "exclude" in _err()
    a.flags = _lib.TGX_CSR_NONDECREASING
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "needs TGX_CSR_EVENTS_BY_CALL" in _err()
    a.flags = _lib.TGX_CSR_EVENTS_BY_CALL | _lib.TGX_CSR_NONDECREASING
    a.num_calls = 2
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "call_starts" in _err()
    a.num_calls = -1
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "call_starts" in _err()
    a.num_calls, a.num_entries = 0, 5
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "even" in _err()
    a.flags = 8
    assert L.tgx_csr_build(ctypes.byref(a), None) == 1 and "unknown flags" in _err()
    # workspace: keys, values and node keys double-buffered, plus the digit counts
    assert L.tgx_csr_build_workspace_size(1 << 20) >= (1 << 20) * 32 + 256 * 512 * 4
    assert L.tgx_csr_build_workspace_size(0) > 0


def test_csr_scan_argument_checks():
    L = _lib.lib()
    ws = L.tgx_csr_scan_workspace_size()
    assert ws >= 1024 * 32
    assert L.tgx_csr_scan(8, 8, 8, 0, None, 0, 8, 8, ws, None) == 1 and "positive" in _err()
    assert L.tgx_csr_scan(8, 8, 8, 5, None, -1, 8, 8, ws, None) == 1 and "num_calls" in _err()
    assert L.tgx_csr_scan(8, None, 8, 5, None, 0, 8, 8, ws, None) == 1 and "NULL" in _err()
    assert L.tgx_csr_scan(8, 8, 8, 5, None, 2, 8, 8, ws, None) == 1 and "call_starts" in _err()
    assert L.tgx_csr_scan(8, 8, 8, 5, None, 0, None, 8, ws, None) == 1 and "NULL" in _err()
    assert L.tgx_csr_scan(8, 8, 8, 5, 8, 1, 8, 8, ws - 1, None) == 1 and "workspace" in _err()
    assert L.tgx_csr_scan(8, 8, 8, 5, 8, 1, 8, None, ws, None) == 1 and "workspace" in _err()


def test_negpool_argument_checks():
    L = _lib.lib()
    assert L.tgx_negpool_update(None, None, 10, 4, 8, 8, 1, 0, 0, 8, 1 << 20, None, 0, None, None) == 1
    assert L.tgx_negpool_update(8, 8, 0, 4, 8, 8, 1, 0, 0, 8, 1 << 20, None, 0, None, None) == 3
    assert L.tgx_negpool_update(8, 8, 10, 0, 8, 8, 1, 0, 0, 8, 1 << 20, None, 0, None, None) == 3
    assert "pool_size" in _err()
    assert L.tgx_negpool_update(8, 8, 10, 4, None, 8, 1, 0, 0, 8, 1 << 20, None, 0, None, None) == 1
    assert L.tgx_negpool_update(8, 8, 10, 4, 8, 8, 100, 0, 0, 8, 16, None, 0, None, None) == 1
    assert "workspace" in _err()
    # the cell table: its size, and 256-byte alignment (checked before any launch)
    sz = L.tgx_negpool_scratch_size()
    assert sz == 65536 * 12
    assert L.tgx_negpool_update(8, 8, 10, 4, 8, 8, 100, 0, 0, 256, 1 << 20, 256, sz - 1, None, None) == 1
    assert "scratch" in _err()
    assert L.tgx_negpool_update(8, 8, 10, 4, 8, 8, 100, 0, 0, 256, 1 << 20, 264, sz, None, None) == 1
    assert "aligned" in _err()
    assert L.tgx_negpool_update(8, 8, 10, 4, 8, 8, 0, 0, 0, None, 0, None, 0, None, None) == 0  # empty batch
    assert L.tgx_negpool_sample(8, 8, 10, 4, None, 5, 0, 0, 8, None, None) == 1
    assert L.tgx_negpool_sample(8, 8, 10, 4, 8, -1, 0, 0, 8, None, None) == 1
    # keys, values, composite keys and values double-buffered, plus digit counts
    assert L.tgx_negpool_update_workspace_size(1 << 16) >= (1 << 16) * 40


def test_co_occurrence_argument_checks():
    L = _lib.lib()
    assert L.tgx_co_occurrence(8, 8, None, None, -1, 4, 8, 8, None, None) == 1
    assert L.tgx_co_occurrence(8, 8, None, None, 4, 5000, 8, 8, None, None) == 3
    assert L.tgx_co_occurrence(None, None, None, None, 0, 4, None, None, None, None) == 0
    assert L.tgx_co_occurrence(None, None, None, None, 4, 4, None, None, None, None) == 1


def test_last_error_is_per_thread():
    L = _lib.lib()
    L.tgx_co_occurrence(8, 8, None, None, -1, 4, 8, 8, None, None)
    main_msg = _err()
    seen = []

    def other():
        L.tgx_co_occurrence(8, 8, None, None, 4, 5000, 8, 8, None, None)
        seen.append(_lib.lib().tgx_last_error().decode())

    th = threading.Thread(target=other)
    th.start()
    th.join()
    assert "negative" in main_msg and "above 4096" in seen[0]
    assert _err() == main_msg


def test_event_groups_with_a_tiled_tail():
    """TGX_PLAN_EVENTS with event_query_groups = 2: the first two query groups
    (src, dst) form one pair per event, and the remaining groups' queries follow
    in workgroups of `group` consecutive queries, so a small launch can split
    each query over more wavefronts."""
    L = _lib.lib()
    b, K = 200, 32
    ring = _lib.TgxRing(num_nodes=10, slots=32, feat_dim=172, feat_dtype=0, ids=16, times=16,
                        feats=16, write_pos=16)

    def args(eqg, per_neg=1):
        groups = [(b, 1), (b, 1), (b * per_neg, per_neg)]
        a = _lib.TgxRecentArgs(k=K, plan_mode=_lib.TGX_PLAN_EVENTS, num_groups=b,
                               num_queries=sum(c for c, _ in groups), out_ids=16, out_times=16,
                               out_mask=16, out_feats=16, d_t=100, te_w=16, out_te=16,
                               co_mode=_lib.TGX_CO_FREQ, co_a=16, co_c=16, event_query_groups=eqg)
        a.group = 2 if eqg == 2 else 2 + per_neg
        a.num_query_groups = len(groups)
        for g, (cnt, per) in enumerate(groups):
            a.query_groups[g].nodes = 16
            a.query_groups[g].times = 16
            a.query_groups[g].count = cnt
            a.query_groups[g].times_per = per
        return a

    rc, full = _shape(ctypes.byref(ring), None, args(0))
    assert rc == 0, _err()
    assert full[0] == b and full[5] == 3 and full[4] == 2  # 3 queries x split 2 per workgroup
    rc, tail = _shape(ctypes.byref(ring), None, args(2))
    assert rc == 0, _err()
    assert tail[4] == 4 and tail[5] == 2 and tail[1] == 64 * 8  # 2 queries x split 4
    assert tail[0] == b + b // 2  # the pairs, then 200 negatives two per workgroup
    rc, tail3 = _shape(ctypes.byref(ring), None, args(2, per_neg=3))
    assert rc == 0 and tail3[0] == b + (3 * b + 1) // 2
    a = args(4)
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "event_query_groups" in _err()
    a = args(2)
    a.group = 3  # must be the event groups' sum of times_per
    assert L.tgx_recent(ctypes.byref(ring), None, ctypes.byref(a), None) == 1 and "times_per" in _err()
