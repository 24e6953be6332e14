"""ctypes binding of libtgx.so (the HIP/gfx950 library behind the C ABI in include/tgx.h).

The library is loaded lazily on first use.  There is no fallback: if the shared
object is missing or cannot be loaded, every call raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent.parent / "_lib" / "libtgx.so"

TGX_OK = 0
TGX_F32 = 0
TGX_BF16 = 1
TGX_QG_NODES_I32 = 1
TGX_DT_DYGFORMER = 0
TGX_DT_TGN = 1
TGX_CO_NONE = 0
TGX_CO_FREQ = 1
TGX_CO_DYGFORMER = 2
TGX_PLAN_TILES = 0
TGX_PLAN_EVENTS = 1
TGX_PLAN_LIST = 2
TGX_ABI_VERSION = 17
TGX_STATUS_WORDS = 8
TGX_ST_BAD_EVENT_NODE = 0
TGX_ST_KEY_COLLISION = 1
TGX_ST_BAD_QUERY_NODE = 2
TGX_MAX_SLOTS = 64
TGX_MAX_K = 512
TGX_MAX_GROUP = 8
TGX_MAX_DT = 512

c_i32, c_i64, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class TgxRing(ctypes.Structure):
    _fields_ = [("num_nodes", c_i64), ("slots", c_i32), ("feat_dim", c_i32),
                ("feat_dtype", c_i32), ("reserved", c_i32), ("ids", c_vp), ("times", c_vp),
                ("feats", c_vp), ("write_pos", c_vp), ("eids", c_vp), ("scratch", c_vp)]


class TgxCsr(ctypes.Structure):
    _fields_ = [("num_nodes", c_i64), ("num_entries", c_i64), ("feat_dim", c_i32),
                ("feat_dtype", c_i32), ("offsets", c_vp), ("ids", c_vp), ("times", c_vp),
                ("feats", c_vp), ("eids", c_vp), ("max_time", ctypes.c_double)]


TGX_MAX_QUERY_GROUPS = 4


class TgxQueryGroup(ctypes.Structure):
    _fields_ = [("nodes", c_vp), ("times", c_vp), ("count", c_i64), ("times_per", c_i32),
                ("flags", c_i32), ("valid", c_vp)]


class TgxRecentArgs(ctypes.Structure):
    _fields_ = [("nodes", c_vp), ("times", c_vp), ("num_queries", c_i64), ("k", c_i32),
                ("plan", c_vp), ("group", c_i32), ("plan_mode", c_i32), ("num_groups", c_i64),
                ("out_ids", c_vp), ("out_times", c_vp), ("out_feats", c_vp), ("out_mask", c_vp),
                ("out_eids", c_vp),
                ("d_t", c_i32), ("te_w", c_vp), ("te_b", c_vp), ("dt_mode", c_i32), ("out_te", c_vp),
                ("co_mode", c_i32), ("co_a", c_vp), ("co_c", c_vp), ("co_pair", c_vp),
                ("status", c_vp), ("num_query_groups", c_i32),
                ("query_groups", TgxQueryGroup * TGX_MAX_QUERY_GROUPS),
                ("timing_start", c_vp), ("timing_stop", c_vp),
                ("append_src", c_vp), ("append_dst", c_vp), ("append_time", c_vp),
                ("append_b", c_i64), ("append_workspace", c_vp),
                ("append_workspace_bytes", ctypes.c_size_t),
                ("event_query_groups", c_i32), ("te_bound_w", ctypes.c_float),
                ("te_bound_b", ctypes.c_float)]


class TgxCsrBuildArgs(ctypes.Structure):
    _fields_ = [("num_nodes", c_i64), ("num_entries", c_i64), ("from_", c_vp), ("to", c_vp),
                ("time", c_vp), ("event", c_vp), ("feats", c_vp), ("num_events", c_i64),
                ("feat_dim", c_i32), ("feat_dtype", c_i32), ("out_offsets", c_vp),
                ("out_ids", c_vp), ("out_times", c_vp), ("out_feats", c_vp), ("out_eids", c_vp),
                ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t), ("status", c_vp),
                ("flags", ctypes.c_uint32), ("call_starts", c_vp), ("num_calls", c_i64)]


TGX_CSR_EVENT_PAIRS = 1
TGX_CSR_EVENTS_BY_CALL = 2
TGX_CSR_NONDECREASING = 4


# every symbol include/tgx.h declares, with its ctypes signature
SIGNATURES = {
    "tgx_ring_append": (c_i32, [ctypes.POINTER(TgxRing), c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                                c_vp, ctypes.c_size_t, c_vp, c_vp]),
    "tgx_ring_plan": (c_i32, [ctypes.POINTER(TgxRing), c_vp, c_vp, c_vp, c_i64, c_vp, ctypes.c_size_t,
                              c_vp]),
    "tgx_ring_commit": (c_i32, [ctypes.POINTER(TgxRing), c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                                c_vp, ctypes.c_size_t, c_vp, c_vp]),
    "tgx_ring_discard": (c_i32, [ctypes.POINTER(TgxRing), c_vp, c_vp, c_i64, c_vp, ctypes.c_size_t,
                                 c_vp]),
    "tgx_ring_append_workspace_size": (ctypes.c_size_t, [c_i64]),
    "tgx_ring_append_static": (c_i32, [ctypes.POINTER(TgxRing), c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                                       c_vp, c_vp]),
    "tgx_ring_append_static_max_bytes": (ctypes.c_size_t, []),
    "tgx_ring_scratch_size": (ctypes.c_size_t, [c_i64]),
    "tgx_recent": (c_i32, [ctypes.POINTER(TgxRing), ctypes.POINTER(TgxCsr),
                           ctypes.POINTER(TgxRecentArgs), c_vp]),
    "tgx_recent_launch_shape": (c_i32, [ctypes.POINTER(TgxRing), ctypes.POINTER(TgxCsr),
                                        ctypes.POINTER(TgxRecentArgs), ctypes.POINTER(c_i64)]),
    "tgx_co_occurrence": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "tgx_csr_build": (c_i32, [ctypes.POINTER(TgxCsrBuildArgs), c_vp]),
    "tgx_csr_build_workspace_size": (ctypes.c_size_t, [c_i64]),
    "tgx_csr_scan": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, ctypes.c_size_t, c_vp]),
    "tgx_csr_scan_workspace_size": (ctypes.c_size_t, []),
    "tgx_negpool_update_workspace_size": (ctypes.c_size_t, [c_i64]),
    "tgx_negpool_scratch_size": (ctypes.c_size_t, []),
    "tgx_negpool_update": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp, c_vp, c_i64, ctypes.c_uint64,
                                   ctypes.c_uint64, c_vp, ctypes.c_size_t, c_vp, ctypes.c_size_t, c_vp, c_vp]),
    "tgx_negpool_sample": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp, c_i64, ctypes.c_uint64,
                                   ctypes.c_uint64, c_vp, c_vp, c_vp]),
    "tgx_negpool_update_draws": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp, c_vp, c_i64, c_vp, c_vp,
                                         c_vp, ctypes.c_size_t, c_vp, c_vp]),
    "tgx_negpool_sample_draws": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp,
                                         c_vp]),
    "tgx_last_error": (ctypes.c_char_p, []),
    "tgx_abi_version": (c_i32, []),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it is not built or not loadable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = os.environ.get("TGX_LIB", str(LIB_PATH))
        if not Path(path).exists():
            raise RuntimeError(
                f"libtgx.so not found at {path}: build it with `python -m tgengine_amd.build` "
                "(tgengine_amd has no CPU fallback)")
        try:
            handle = ctypes.CDLL(path)
        except OSError as exc:  # pragma: no cover - depends on the ROCm install
            raise RuntimeError(f"cannot load {path}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.tgx_abi_version() != TGX_ABI_VERSION:
            raise RuntimeError("libtgx ABI version mismatch")
        _lib = handle
        return _lib


def check(rc: int, what: str) -> None:
    if rc != TGX_OK:
        msg = lib().tgx_last_error()
        raise RuntimeError(f"{what} failed (code {rc}): {msg.decode() if msg else ''}")


def ptr(t) -> int:
    """Device pointer of a tensor, or 0 for None."""
    return 0 if t is None else t.data_ptr()
