"""TemporalGraph: the drop-in for tgengine/core/temporal_graph.py:31-564 on MI355X.

Same lifecycle and semantics as the reference:

1. Build: ``advance()`` before the first query accumulates events on the host.
2. Freeze: the first query (or ``freeze_csr()``) sorts them into an immutable
   CSR on the device (temporal_graph.py:133-181).
3. Stream: every ``advance()`` after the freeze goes to the per-node ring of
   ``buffer_size`` slots (allocated lazily, :89-102) through the HIP kernel
   ``tgx_ring_append`` (reference ``_append_overflow`` :351-387).

``recent`` merges the CSR window with the valid ring slots in one HIP launch
(``tgx_recent``; reference :183-349).  Every device computation goes through
libtgx.so on the caller's current stream; there is no CPU fallback and a
missing library raises.

Extensions (keyword-only, defaults match the reference):
``feat_dtype`` (torch.float32 or torch.bfloat16 ring storage) and
``track_edge_ids`` (keep the global event index of every ring/CSR entry).
"""
from __future__ import annotations

import ctypes
import struct
import threading
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .batch import NeighborData

try:
    from tgengine_amd import _tgx_host
except ImportError as _exc:  # pragma: no cover - the product path has no fallback
    _tgx_host = None
    _HOST_ERR = _exc

_DTYPES = {torch.float32: _lib.TGX_F32, torch.bfloat16: _lib.TGX_BF16}


@dataclass
class Snapshot:
    """Ring state for eval restore (reference temporal_graph.py:17-28); the CSR is immutable."""

    overflow_ids: Tensor
    overflow_times: Tensor
    overflow_feats: Tensor
    overflow_write_pos: Tensor
    num_edges: int
    overflow_eids: Optional[Tensor] = None


class _PlanView:
    """Read-only view of the pending ring plan (its stream), for diagnostics."""

    __slots__ = ("stream",)

    def __init__(self, stream: int):
        self.stream = stream


try:
    _raw_stream = torch._C._cuda_getCurrentRawStream  # (device_index) -> hipStream_t as int
except AttributeError:  # pragma: no cover - older torch
    _raw_stream = None


_WS_SIZES: dict = {}


def _ws_size(b: int) -> int:
    """tgx_ring_append_workspace_size(b), remembered per batch length."""
    n = _WS_SIZES.get(b)
    if n is None:
        n = _WS_SIZES[b] = int(_lib.lib().tgx_ring_append_workspace_size(b))
    return n


def _stream_handle(device: torch.device) -> int:
    """hipStream_t of the caller's current stream on ``device``."""
    if _raw_stream is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _as(t: Tensor, dtype: torch.dtype, device: torch.device) -> Tensor:
    """``t`` as a contiguous ``dtype`` tensor on ``device`` (no copy when it already is)."""
    if t.dtype == dtype and t.device == device and t.is_contiguous():
        return t
    return t.to(device, dtype).contiguous()


def _host():
    """The host-glue extension; raises when it was not built (no fallback)."""
    if _tgx_host is None:
        raise RuntimeError("tgengine_amd._tgx_host is not built: run `python -m tgengine_amd.build` "
                           f"({_HOST_ERR})")
    return _tgx_host


class TemporalGraph:
    PADDING_ID: int = -1

    def __init__(self, num_nodes: int, edge_feat_dim: int = 172,
                 device: str | torch.device = "cuda", overflow_size: int = 64,
                 buffer_size: Optional[int] = None, use_triton: bool = True, *,
                 feat_dtype: torch.dtype = torch.float32, track_edge_ids: bool = False):
        if buffer_size is not None:
            overflow_size = buffer_size
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError(
                f"tgengine_amd.TemporalGraph runs on a ROCm GPU (device='cuda'), got {device!r}; "
                "there is no CPU path")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        _lib.lib()  # raises when libtgx.so is missing
        if feat_dtype not in _DTYPES:
            raise TypeError(f"feat_dtype must be torch.float32 or torch.bfloat16, got {feat_dtype}")
        if not 1 <= int(overflow_size) <= _lib.TGX_MAX_SLOTS:
            raise ValueError(f"buffer_size must be in [1, {_lib.TGX_MAX_SLOTS}], got {overflow_size}")
        if not 0 < int(num_nodes) < 2 ** 31:
            raise ValueError(f"num_nodes must be in [1, 2^31), got {num_nodes}")
        self._use_triton = use_triton  # accepted for signature compatibility
        self.num_nodes = int(num_nodes)
        self.edge_feat_dim = int(edge_feat_dim)
        self.overflow_size = int(overflow_size)
        self.feat_dtype = feat_dtype
        self.track_edge_ids = bool(track_edge_ids)
        self._num_edges = 0

        # pre-freeze events, appended in advance() order to device buffers that
        # grow by doubling: src, dst (int64), time (float64), feat rows (made on
        # the first batch with features, zero rows before it); the event index in
        # them is the global edge id.  _build_starts: first event of each call
        self._build: dict = {}
        self._build_n = 0
        self._build_starts: list = []
        self._frozen = False
        self._offsets: Optional[Tensor] = None
        self._nbr_ids: Optional[Tensor] = None
        self._nbr_times: Optional[Tensor] = None
        self._nbr_feats: Optional[Tensor] = None
        self._nbr_eids: Optional[Tensor] = None
        self._csr_max_time = float("inf")  # largest non-NaN CSR time (a search hint)
        self._csr_time_sorted = False  # freeze_csr took the event-pair build
        self._csr_build_mode = ""  # freeze_csr's build: "pairs", "runs" or "sort"

        self._ov_ids: Optional[Tensor] = None
        self._ov_times: Optional[Tensor] = None
        self._ov_feats: Optional[Tensor] = None
        self._ov_write_pos: Optional[Tensor] = None
        self._ov_eids: Optional[Tensor] = None
        self._ov_scratch: Optional[Tensor] = None

        self._status = torch.zeros(_lib.TGX_STATUS_WORDS, dtype=torch.int32, device=self.device)
        self._ws: Optional[Tensor] = None
        # the ring update planned ahead of its advance() (see plan_append): the
        # extension's PlanSlot of the current ring, with the plan workspace; the
        # lock serialises the multi-step paths (discard, re-plan) between threads
        self._slot = None
        self._plan_lock = threading.Lock()
        self._ring_struct: Optional[_lib.TgxRing] = None
        self._csr_struct: Optional[_lib.TgxCsr] = None
        # bumped whenever the ring or CSR arrays (and so their C structs) change:
        # launch contexts cached by a DataPipeline are rebuilt when it moves
        self._gen = 0
        # optional object whose events() returns a (start, stop) pair of raw
        # hipEvent_t handles (or (0, 0)); each tgx_recent launch records the
        # kernel's own start and end on them
        self.kernel_timer = None

    # ------------------------------------------------------------------ ring
    def _ensure_overflow(self) -> None:
        if self._ov_ids is not None:
            return
        N, B, d = self.num_nodes, self.overflow_size, self.edge_feat_dim
        dev = self.device
        self._ov_ids = torch.full((N, B), self.PADDING_ID, dtype=torch.int32, device=dev)
        self._ov_times = torch.zeros((N, B), dtype=torch.float64, device=dev)
        self._ov_feats = torch.zeros((N, B, d), dtype=self.feat_dtype, device=dev)
        self._ov_write_pos = torch.zeros(N, dtype=torch.int64, device=dev)
        if self.track_edge_ids:
            self._ov_eids = torch.full((N, B), -1, dtype=torch.int64, device=dev)
        # per-node counters of tgx_ring_append (zero between calls)
        nscr = int(_lib.lib().tgx_ring_scratch_size(N)) // 4
        self._ov_scratch = torch.zeros(nscr, dtype=torch.int32, device=dev)
        self._ring_struct = None
        self._slot = _host().PlanSlot(ctypes.addressof(self._ring()), self._status, self.edge_feat_dim,
                                      self.feat_dtype)
        self._gen += 1

    def _ring(self) -> Optional[_lib.TgxRing]:
        if self._ov_ids is None:
            return None
        if self._ring_struct is None:
            self._ring_struct = _lib.TgxRing(
                num_nodes=self.num_nodes, slots=self.overflow_size, feat_dim=self.edge_feat_dim,
                feat_dtype=_DTYPES[self.feat_dtype], reserved=0,
                ids=self._ov_ids.data_ptr(), times=self._ov_times.data_ptr(),
                feats=self._ov_feats.data_ptr(), write_pos=self._ov_write_pos.data_ptr(),
                eids=_lib.ptr(self._ov_eids), scratch=self._ov_scratch.data_ptr())
        return self._ring_struct

    def _csr(self) -> Optional[_lib.TgxCsr]:
        if not self._frozen:
            return None
        if self._csr_struct is None:
            self._csr_struct = _lib.TgxCsr(
                num_nodes=self.num_nodes, num_entries=int(self._nbr_ids.shape[0]),
                feat_dim=self.edge_feat_dim, feat_dtype=_DTYPES[self.feat_dtype],
                offsets=self._offsets.data_ptr(), ids=_lib.ptr(self._nbr_ids),
                times=_lib.ptr(self._nbr_times), feats=_lib.ptr(self._nbr_feats),
                eids=_lib.ptr(self._nbr_eids), max_time=self._csr_max_time)
        return self._csr_struct

    def _feat_in(self, edge_feat: Optional[Tensor], b: int) -> Optional[Tensor]:
        if edge_feat is None:
            return None
        if edge_feat.dim() != 2 or edge_feat.shape[0] != b or edge_feat.shape[1] != self.edge_feat_dim:
            raise ValueError(f"edge_feat must be ({b}, {self.edge_feat_dim}), got {tuple(edge_feat.shape)}")
        if edge_feat.dtype != self.feat_dtype:
            if self.feat_dtype == torch.bfloat16 and edge_feat.dtype == torch.float32:
                edge_feat = edge_feat.to(torch.bfloat16)  # round to nearest even
            else:
                raise RuntimeError("Index put requires the source and destination dtypes match, "
                                   f"got {self.feat_dtype} for the ring and {edge_feat.dtype} for edge_feat")
        return _as(edge_feat, self.feat_dtype, self.device)

    def _grown(self, old: Optional[Tensor], nbytes: int) -> Tensor:
        """A workspace of at least nbytes.  Launches on several streams (the
        prefetch stream's plan, the caller's commit) may still read the one it
        replaces, so the device drains before that is released; workspaces only
        grow, so this happens a few times per graph at most."""
        if old is not None and old.numel() >= nbytes:
            return old
        if old is not None:
            torch.cuda.synchronize(self.device)
        return torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=self.device)

    def _workspace(self, nbytes: int) -> Tensor:
        self._ws = self._grown(self._ws, nbytes)
        return self._ws

    # ------------------------------------------------------------------ planned updates
    def _plannable(self, src: Tensor, dst: Tensor, time: Tensor) -> bool:
        """Whether the batch can be planned ahead: a frozen graph on the GPU whose
        ring exists, and int64 / float64 contiguous 1-D device inputs."""
        if not self._frozen or self._ov_ids is None or self.device.type != "cuda":
            return False
        b = int(src.shape[0])
        return (b > 0 and dst.shape[0] == b and time.shape[0] == b and src.dim() == 1
                and dst.dim() == 1 and time.dim() == 1 and src.dtype == torch.int64
                and dst.dtype == torch.int64 and time.dtype == torch.float64
                and all(t.device == self.device and t.is_contiguous() for t in (src, dst, time)))

    def _plan_workspace(self, b: int) -> Tensor:
        slot = self._slot
        ws = slot.workspace()
        need = _ws_size(b)
        if ws is None or ws.numel() < need:
            ws = self._grown(ws, need)
            slot.set_workspace(ws)
        return ws

    @property
    def _plan(self) -> Optional[_PlanView]:
        """The pending ring plan's stream, or None when no plan is pending."""
        slot = self._slot
        if slot is None or not slot.pending():
            return None
        return _PlanView(slot.stream())

    def _order_after(self, stream: int) -> int:
        """Raw handle of the current stream, made to wait for ``stream`` first when
        that is another stream."""
        cur = _stream_handle(self.device)
        if stream != cur:
            torch.cuda.current_stream(self.device).wait_stream(
                torch.cuda.ExternalStream(stream, device=self.device))
        return cur

    def plan_append(self, src: Tensor, dst: Tensor, time: Tensor) -> bool:
        """Enqueue the first half of the ring update of a batch that advance()
        will receive next (tgx_ring_plan, on the current stream).

        The plan (per-node counts and entry lists) reads only src/dst/time and
        writes only the ring's scratch, never the ring arrays, so queries may run
        between the plan and its advance.  DataPipeline.prepare runs the same
        plan inside its gather launch.  advance() commits the plan when it
        receives the very same src/dst/time tensors unchanged (same storage,
        shape, dtype and version counter), otherwise it discards it and runs the
        whole update.  Returns whether a plan was enqueued."""
        if not self._plannable(src, dst, time):
            return False
        with self._plan_lock:
            self._discard_plan()  # an earlier plan nobody advanced
            stream = _stream_handle(self.device)
            ws = self._plan_workspace(int(src.shape[0]))
            _host().ring_plan(ctypes.addressof(self._ring()), src, dst, time, ws, stream)
            self._slot.record(src, dst, time, stream)
        return True

    def _adopt_plan(self, stream) -> None:
        """The caller has ordered ``stream`` (a torch stream) after the pending
        plan's stream: a commit or discard on ``stream`` needs no further wait."""
        if self._slot is not None:
            self._slot.set_stream(stream.cuda_stream)

    def _discard_plan(self) -> None:
        """Discard the pending plan, if any, on the current stream (ordered after
        the plan's stream)."""
        plan = self._slot.take() if self._slot is not None else None
        if plan is None:
            return
        src, dst, _, pstream = plan
        stream = self._order_after(pstream)
        _host().ring_discard(ctypes.addressof(self._ring()), src, dst, self._slot.workspace(), stream)

    def _drop_plan(self) -> None:
        """Discard a pending plan (before the ring or its scratch is replaced)."""
        with self._plan_lock:
            self._discard_plan()

    def advance(self, src: Tensor, dst: Tensor, time: Tensor,
                edge_feat: Optional[Tensor] = None) -> None:
        """Append a batch of undirected events (reference temporal_graph.py:104-131)."""
        slot = self._slot
        if slot is not None:
            # the planned batch, on the plan's stream, with a ready feature block:
            # one call commits it
            n = slot.commit(src, dst, time, edge_feat, self._num_edges)
            if n:
                self._num_edges += n
                return
        b = int(src.shape[0])
        if dst.shape[0] != b or time.shape[0] != b:
            raise ValueError("src, dst and time must have the same length")
        if slot is not None and slot.pending():
            with self._plan_lock:
                if slot.matches(src, dst, time):
                    try:
                        feat = self._feat_in(edge_feat, b)
                    except Exception:
                        self._discard_plan()
                        raise
                    _, _, _, pstream = slot.take()
                    stream = self._order_after(pstream)
                    _host().ring_commit(ctypes.addressof(self._ring()), src, dst, time, feat,
                                        self._num_edges, slot.workspace(), self._status, stream)
                    self._num_edges += b
                    return
                self._discard_plan()
        if not self._frozen:
            # the values at call time, copied into the device event buffers (the
            # reference copies them into host lists, temporal_graph.py:110-122)
            if b > 0:
                self._build_append(src, dst, time, self._feat_in(edge_feat, b), b)
        else:
            self._ensure_overflow()
            if b > 0:
                self._append_ring(src, dst, time, edge_feat, b)
        self._num_edges += b

    def _append_ring(self, src, dst, time, edge_feat, b: int) -> None:
        feat = self._feat_in(edge_feat, b)
        need = int(_lib.lib().tgx_ring_append_workspace_size(b))
        ws = self._workspace(need)
        _host().ring_append(ctypes.addressof(self._ring()), src, dst, time, feat, self._num_edges,
                            ws, self._status, _stream_handle(self.device))

    # ------------------------------------------------------------------ CSR
    def _build_append(self, src: Tensor, dst: Tensor, time: Tensor, feat: Optional[Tensor],
                      b: int) -> None:
        """Copy one pre-freeze batch into the event buffers (grown by doubling)."""
        dev, d = self.device, self.edge_feat_dim
        n0 = self._build_n
        n1 = n0 + b
        bufs = self._build
        cap = int(bufs["src"].shape[0]) if bufs else 0
        if n1 > cap:
            cap = max(n1, 2 * cap, 1 << 12)
            grown = {"src": torch.empty(cap, dtype=torch.int64, device=dev),
                     "dst": torch.empty(cap, dtype=torch.int64, device=dev),
                     "time": torch.empty(cap, dtype=torch.float64, device=dev)}
            if "feat" in bufs:
                grown["feat"] = torch.empty((cap, d), dtype=self.feat_dtype, device=dev)
            for k, v in bufs.items():
                grown[k][:n0].copy_(v[:n0])
            self._build = bufs = grown
        bufs["src"][n0:n1].copy_(src.detach().reshape(-1))
        bufs["dst"][n0:n1].copy_(dst.detach().reshape(-1))
        bufs["time"][n0:n1].copy_(time.detach().reshape(-1))
        if feat is not None and d > 0 and "feat" not in bufs:
            bufs["feat"] = torch.empty((cap, d), dtype=self.feat_dtype, device=dev)
            bufs["feat"][:n0].zero_()
        if "feat" in bufs:
            if feat is None:
                bufs["feat"][n0:n1].zero_()
            else:
                bufs["feat"][n0:n1].copy_(feat)
        self._build_starts.append(n0)
        self._build_n = n1

    def freeze_csr(self) -> None:
        """Build the frozen CSR on the device from the pre-freeze events
        (reference :133-181), with tgx_csr_build.

        Build order per advance() call is [src->dst ..., dst->src ...]; entries
        are sorted stably by time, then stably by node, so a node's entries are
        time-ascending with ties in build order.  When the event times increase
        strictly within every call and never decrease across calls (a
        time-ordered stream), that time order is already the events' own order
        with each event's two entries side by side, and the build sorts by node
        only (TGX_CSR_EVENT_PAIRS).  When they only never decrease (ties), the
        time order is, run by run of equal times within a call, the run's
        src->dst entries then its dst->src entries, and again only the node
        passes run (TGX_CSR_EVENTS_BY_CALL | TGX_CSR_NONDECREASING).  Otherwise
        the device forms the build order from the events and the calls' first
        events and sorts it by time first (TGX_CSR_EVENTS_BY_CALL).
        """
        N, d, dev = self.num_nodes, self.edge_feat_dim, self.device
        E = self._build_n
        n = 2 * E
        self._offsets = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        self._nbr_ids = torch.empty(n, dtype=torch.int32, device=dev)
        self._nbr_times = torch.empty(n, dtype=torch.float64, device=dev)
        self._nbr_feats = torch.empty((n, d), dtype=self.feat_dtype, device=dev)
        self._nbr_eids = torch.empty(n, dtype=torch.int64, device=dev) if self.track_edge_ids else None
        if n > 0:
            bufs = self._build
            src, dst, tt = bufs["src"][:E], bufs["dst"][:E], bufs["time"][:E]
            feats = bufs["feat"][:E] if "feat" in bufs else None
            # one device round trip (tgx_csr_scan): node range, whether the stream
            # is time-ordered, and the largest non-NaN time
            L = _lib.lib()
            ws = torch.empty(max(int(L.tgx_csr_build_workspace_size(n)), int(L.tgx_csr_scan_workspace_size())),
                             dtype=torch.uint8, device=dev)
            call_starts = torch.tensor(self._build_starts, dtype=torch.int64).to(dev)
            scan = torch.empty(4, dtype=torch.int64, device=dev)
            _lib.check(L.tgx_csr_scan(src.data_ptr(), dst.data_ptr(), tt.data_ptr(), E, call_starts.data_ptr(),
                                      call_starts.numel(), scan.data_ptr(), ws.data_ptr(), ws.numel(),
                                      _stream_handle(dev)), "tgx_csr_scan")
            lo, hi, order, tbits = scan.cpu().tolist()
            self._csr_max_time = struct.unpack("<d", struct.pack("<q", tbits))[0]
            if lo < 0 or hi >= N:
                raise IndexError("advance() got node ids outside [0, num_nodes)")
            # which build runs (diagnostics): the events in pairs (strictly
            # increasing times within each call), runs of equal times of a
            # non-decreasing stream, or the build order sorted by time
            self._csr_time_sorted = order == 2
            self._csr_build_mode = ("sort", "runs", "pairs")[order]
            if order == 2:
                flags = _lib.TGX_CSR_EVENT_PAIRS
            else:
                flags = _lib.TGX_CSR_EVENTS_BY_CALL | (_lib.TGX_CSR_NONDECREASING if order == 1 else 0)
            a = _lib.TgxCsrBuildArgs(
                num_nodes=N, num_entries=n, from_=src.data_ptr(), to=dst.data_ptr(),
                time=tt.data_ptr(), event=None, call_starts=call_starts.data_ptr(),
                num_calls=call_starts.numel(),
                feats=feats.data_ptr() if feats is not None else None,
                num_events=E if feats is not None else 0,
                feat_dim=d, feat_dtype=_DTYPES[self.feat_dtype],
                out_offsets=self._offsets.data_ptr(), out_ids=self._nbr_ids.data_ptr(),
                out_times=self._nbr_times.data_ptr(),
                out_feats=self._nbr_feats.data_ptr() if d > 0 else None,
                out_eids=_lib.ptr(self._nbr_eids), workspace=ws.data_ptr(),
                workspace_bytes=ws.numel(), status=self._status.data_ptr(), flags=flags)
            _lib.check(L.tgx_csr_build(ctypes.byref(a), _stream_handle(dev)), "tgx_csr_build")
        self._frozen = True
        self._build = {}
        self._build_n = 0
        self._build_starts = []
        self._csr_struct = None
        self._gen += 1

    # ------------------------------------------------------------------ queries
    def _query(self, nodes: Optional[Tensor], times: Optional[Tensor], k: int, *,
               groups: Optional[list] = None, plan: Optional[Tensor] = None,
               plan_mode: int = _lib.TGX_PLAN_TILES, group: int = 4,
               num_groups: Optional[int] = None, event_query_groups: int = 0, d_t: int = 0,
               te_w: Optional[Tensor] = None, te_b: Optional[Tensor] = None,
               te_bounds: tuple = (0.0, 0.0),
               dt_mode: int = _lib.TGX_DT_DYGFORMER, co_mode: int = _lib.TGX_CO_NONE,
               want_eids: bool = False, append: Optional[tuple] = None) -> dict:
        """One tgx_recent launch.

        Queries come either as ``nodes``/``times`` or as ``groups``: a list of
        (nodes, times, times_per[, valid]) read in place and concatenated in order
        (int64 or int32 nodes; a False in ``valid`` makes that query padding only).  Returns
        lists of per-group tensors under "ids", "times", "feats", "mask" (bool), and
        "eids" / "te" when asked for, plus "co_a", "co_c", "co_pair" with co-occurrence.
        ``append``: (src, dst, time) of the batch the caller advances next; when it
        can be planned (see plan_append) the same launch also plans its ring update.
        ``event_query_groups``: of an event-major plan, the leading query groups
        grouped per event (0: all); the rest are tiled after them.  -1 picks the
        layout of DataPipeline.prepare (a launch of at most 4096 queries groups only
        the (src, dst) pair per event).  ``te_bounds``: upper bounds of max|te_w| and
        max|te_b| (0, 0: unknown, every encoding takes the full-range reduction).
        """
        if not self._frozen:
            self.freeze_csr()
        k = int(k)
        if not 1 <= k <= _lib.TGX_MAX_K:
            raise ValueError(f"k must be in [1, {_lib.TGX_MAX_K}], got {k}")
        if groups is None:
            if times.shape[0] != nodes.shape[0]:
                raise ValueError("nodes and times must have the same length")
            groups = [(nodes, times, 1)]
        if len(groups) > _lib.TGX_MAX_QUERY_GROUPS:
            raise ValueError(f"at most {_lib.TGX_MAX_QUERY_GROUPS} query groups")
        planned, res = self._gather(groups, k, plan, plan_mode, group, num_groups,
                                    event_query_groups, d_t, (te_w, te_b, te_bounds), dt_mode,
                                    co_mode, want_eids, append)
        nf = 4 + (d_t > 0) + bool(want_eids)
        ng = len(groups)
        out = {"ids": res[0:ng * nf:nf], "times": res[1:ng * nf:nf], "feats": res[2:ng * nf:nf],
               "mask": res[3:ng * nf:nf]}
        if d_t > 0:
            out["te"] = res[4:ng * nf:nf]
        if want_eids:
            out["eids"] = res[nf - 1:ng * nf:nf]
        if co_mode != _lib.TGX_CO_NONE:
            out["co_a"], out["co_c"], out["co_pair"] = res[ng * nf:ng * nf + 3]
        return out

    def _gather(self, groups, k, plan, plan_mode, group, num_groups, ev_groups, d_t, te,
                dt_mode, co_mode, want_eids, append) -> tuple:
        """One tgx_recent launch over checked query groups: the extension's
        (planned, tensors) pair.  When ``append`` is given and the ring exists,
        the launch also plans that batch (see plan_append)."""
        if not self._frozen:
            self.freeze_csr()
        ring = self._ring()
        csr = self._csr()
        ev0 = ev1 = 0
        if self.kernel_timer is not None:
            ev0, ev1 = self.kernel_timer.events()
        stream = _stream_handle(self.device)
        if append is None or ring is None:
            return self._launch_recent(ring, csr, groups, k, plan, plan_mode, group, num_groups,
                                       ev_groups, d_t, te, dt_mode, co_mode, want_eids, ev0,
                                       ev1, None, None, stream)
        # the extension plans the batch when its tensors allow it (int64 / float64
        # contiguous 1-D device tensors of one non-zero length)
        with self._plan_lock:
            self._discard_plan()  # an earlier plan nobody advanced
            ws = self._plan_workspace(int(append[0].shape[0]))
            res = self._launch_recent(ring, csr, groups, k, plan, plan_mode, group, num_groups,
                                      ev_groups, d_t, te, dt_mode, co_mode, want_eids, ev0,
                                      ev1, append, ws, stream)
            if res[0]:
                self._slot.record(append[0], append[1], append[2], stream)
        return res

    def _launch_recent(self, ring, csr, groups, k, plan, plan_mode, group, num_groups, ev_groups,
                       d_t, te, dt_mode, co_mode, want_eids, ev0, ev1, append, ws, stream):
        te_w, te_b, te_bounds = te
        a_src, a_dst, a_time = append if append is not None else (None, None, None)
        gn, gt, gp, gv = [], [], [], []
        for grp in groups:
            gn.append(grp[0])
            gt.append(grp[1])
            gp.append(grp[2])
            if len(grp) > 3:
                gv.append(grp[3])
        if gv and len(gv) != len(groups):
            gv = [grp[3] if len(grp) > 3 else None for grp in groups]
        return _host().recent(
            ctypes.addressof(ring) if ring is not None else 0,
            ctypes.addressof(csr) if csr is not None else 0,
            gn, gt, gp, gv, k, self.edge_feat_dim, self.feat_dtype, plan, int(plan_mode), int(group),
            -1 if num_groups is None else int(num_groups), int(ev_groups), int(d_t), te_w, te_b,
            float(te_bounds[0]), float(te_bounds[1]), int(dt_mode),
            int(co_mode), bool(want_eids), self._status, stream, ev0, ev1,
            a_src, a_dst, a_time, ws)

    def _prepare(self, prep, src: Tensor, dst: Tensor, time: Tensor, neg: Optional[Tensor],
                 neg_src: Optional[Tensor], plan_updates: bool) -> tuple:
        """One DataPipeline 1-hop launch through its configured extension context
        ``prep``: its tensors.  With ``plan_updates`` and a ring, the launch also
        plans the ring update of this batch for the advance() that follows."""
        if not self._frozen:
            self.freeze_csr()
        res = prep.run(src, dst, time, neg, neg_src, plan_updates)
        if res is None:
            # an earlier plan pending on another stream, or a workspace too small:
            # settle the plan state, then launch
            with self._plan_lock:
                self._discard_plan()
                if self._plannable(src, dst, time):
                    self._plan_workspace(int(src.shape[0]))
                res = prep.run(src, dst, time, neg, neg_src, plan_updates)
        return res

    def _structs(self) -> tuple:
        """Addresses of the ring and CSR C structs (0 when absent); stable until
        ``_gen`` changes."""
        ring = self._ring()
        csr = self._csr()
        return (ctypes.addressof(ring) if ring is not None else 0,
                ctypes.addressof(csr) if csr is not None else 0)

    def recent(self, nodes: Tensor, times: Tensor, k: int) -> NeighborData:
        """Most recent k neighbours before each query time (reference :183-280)."""
        o = self._query(nodes, times, k, want_eids=self.track_edge_ids)
        return NeighborData(neighbor_ids=o["ids"][0], timestamps=o["times"][0],
                            edge_feats=o["feats"][0], mask=o["mask"][0],
                            edge_ids=o["eids"][0] if "eids" in o else None)

    def recent_2hop(self, nodes: Tensor, times: Tensor, k1: int, k2: int) -> NeighborData:
        """1-hop and 2-hop neighbours (reference :397-473), in two launches like the
        reference's CUDA path (hop 1, then one query per hop-1 slot): the 2-hop query
        of slot (b, i) is (hop1 id, hop1 time), read in place from the hop-1 outputs;
        slots under an invalid hop-1 neighbour come out as padding."""
        hop1 = self.recent(nodes, times, k1)
        N, K1 = hop1.neighbor_ids.shape
        o = self._query(None, None, k2, groups=[(hop1.neighbor_ids.reshape(-1), hop1.timestamps.reshape(-1),
                                                 1, hop1.mask.reshape(-1))])
        hop1.hop2_ids = o["ids"][0].reshape(N, K1, k2)
        hop1.hop2_times = o["times"][0].reshape(N, K1, k2)
        hop1.hop2_feats = o["feats"][0].reshape(N, K1, k2, self.edge_feat_dim)
        hop1.hop2_mask = o["mask"][0].reshape(N, K1, k2)
        return hop1

    def co_neighbors(self, src: Tensor, dst: Tensor, times: Tensor, k: int = 32) -> Tensor:
        """(B,) float32 count of src neighbours that also occur among dst's
        neighbours (reference :475-498)."""
        B = int(src.shape[0])
        if B == 0:
            return torch.zeros(0, dtype=torch.float32, device=self.device)
        qt = times.to(self.device, torch.float64)
        # event-major pairs: group p = (src p, dst p)
        o = self._query(None, None, k, groups=[(src.to(self.device, torch.int64), qt, 1),
                                               (dst.to(self.device, torch.int64), qt, 1)],
                        plan_mode=_lib.TGX_PLAN_EVENTS, group=2, num_groups=B,
                        co_mode=_lib.TGX_CO_FREQ)
        return o["co_pair"]

    # ------------------------------------------------------------------ state
    def reset(self) -> None:
        if self._ov_ids is not None:
            self._drop_plan()
        self._frozen = False
        self._build = {}
        self._build_n = 0
        self._build_starts = []
        self._offsets = self._nbr_ids = self._nbr_times = self._nbr_feats = self._nbr_eids = None
        self._csr_max_time = float("inf")
        self._ov_ids = self._ov_times = self._ov_feats = self._ov_write_pos = self._ov_eids = None
        self._ov_scratch = None
        self._ring_struct = None
        self._slot = None
        self._csr_struct = None
        self._gen += 1
        self._num_edges = 0

    def snapshot(self) -> Snapshot:
        """Device clone of the ring state (reference :517-526); allocates the ring if absent."""
        self._ensure_overflow()
        return Snapshot(self._ov_ids.clone(), self._ov_times.clone(), self._ov_feats.clone(),
                        self._ov_write_pos.clone(), self._num_edges,
                        None if self._ov_eids is None else self._ov_eids.clone())

    def restore(self, snap: Snapshot) -> None:
        if self._ov_eids is not None and snap.overflow_eids is None:
            raise ValueError("restore: this graph tracks edge ids and the snapshot holds none; "
                             "its ring edge ids would no longer match the restored slots")
        self._drop_plan()
        self._ov_ids.copy_(snap.overflow_ids)
        self._ov_times.copy_(snap.overflow_times)
        self._ov_feats.copy_(snap.overflow_feats)
        self._ov_write_pos.copy_(snap.overflow_write_pos)
        if self._ov_eids is not None and snap.overflow_eids is not None:
            self._ov_eids.copy_(snap.overflow_eids)
        self._num_edges = snap.num_edges

    @property
    def num_edges(self) -> int:
        return self._num_edges

    def status(self) -> dict:
        """Device diagnostics accumulated by the kernels (synchronises the stream)."""
        s = self._status.cpu().tolist()
        return {"bad_event_nodes": s[_lib.TGX_ST_BAD_EVENT_NODE],
                "key_collisions": s[_lib.TGX_ST_KEY_COLLISION],
                "bad_query_nodes": s[_lib.TGX_ST_BAD_QUERY_NODE]}

    def clear_status(self) -> None:
        self._status.zero_()

    @classmethod
    def from_dataset(cls, src: Tensor, dst: Tensor, time: Tensor, edge_feat: Optional[Tensor],
                     num_nodes: int, device: str = "cuda", **kwargs) -> "TemporalGraph":
        """Replay all events, then freeze (reference :540-564)."""
        d_edge = edge_feat.shape[1] if edge_feat is not None else 172
        graph = cls(num_nodes, edge_feat_dim=d_edge, device=device, **kwargs)
        chunk = 10000
        n = src.shape[0]
        for s in range(0, n, chunk):
            e = min(s + chunk, n)
            graph.advance(src[s:e], dst[s:e], time[s:e],
                          edge_feat[s:e] if edge_feat is not None else None)
        graph.freeze_csr()
        return graph
