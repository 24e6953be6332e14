"""AsyncDataPipeline: the drop-in for tgengine/pipeline/async_pipeline.py:37-143.

A host thread prepares batch i+1 on a side HIP stream while the caller works
on batch i.  Every libtgx launch goes to the *current* stream, so inside the
prefetch thread's ``torch.cuda.stream(side)`` block the kernels are ordered on
the side stream (the reference's native kernels ignore the current stream).

Ordering protocol (unchanged): ``start_prefetch`` makes the side stream wait
for the caller's stream, so it sees the graph after ``advance(i)``; ``get``
joins the thread, re-raises its exception, and makes the caller's stream wait
for the side stream (which also orders the ring plan that prepare() enqueued
there before the caller's ``advance``).
"""
from __future__ import annotations

import dataclasses
import threading
from typing import Optional

import torch

from tgengine_amd.core.batch import PreparedBatch, RawBatch
from tgengine_amd.core.gather_spec import GatherSpec
from tgengine_amd.core.temporal_graph import TemporalGraph


class AsyncDataPipeline:
    def __init__(self, spec: GatherSpec, graph: TemporalGraph, neg_strat, time_encoder=None):
        from tgengine_amd.pipeline import DataPipeline
        self._pipeline = DataPipeline(spec, graph, time_encoder=time_encoder)
        self._neg_strat = neg_strat
        self._graph = graph
        self._prefetch_stream = torch.cuda.Stream(device=graph.device)
        self._thread: Optional[threading.Thread] = None
        self._result = None
        self._exc: Optional[BaseException] = None

    @property
    def spec(self):
        return self._pipeline.spec

    @property
    def graph(self):
        return self._pipeline.graph

    def start_prefetch(self, raw_batch: RawBatch) -> None:
        """Prepare ``raw_batch`` on the side stream; call after ``graph.advance`` of the previous batch.
        A prefetch still running (never collected by ``get``) is joined and dropped first."""
        if self._thread is not None:
            self._thread.join()
            self._thread = None
        self._prefetch_stream.wait_stream(torch.cuda.current_stream(self._graph.device))
        self._result = None
        self._exc = None
        stream = self._prefetch_stream
        neg_strat = self._neg_strat
        pipeline = self._pipeline
        device = self._graph.device

        def _fetch():
            try:
                with torch.cuda.device(device), torch.cuda.stream(stream):
                    neg = neg_strat.sample(raw_batch.src, raw_batch.dst, raw_batch.time,
                                           pipeline.graph, raw_batch.edge_indices)
                    rb = RawBatch(src=raw_batch.src, dst=raw_batch.dst, time=raw_batch.time,
                                  edge_feat=raw_batch.edge_feat, neg=neg,
                                  edge_indices=raw_batch.edge_indices, neg_src=raw_batch.neg_src)
                    self._result = (rb, pipeline.prepare(rb))
            except BaseException as exc:  # re-raised by get()
                self._exc = exc

        self._thread = threading.Thread(target=_fetch, daemon=True)
        self._thread.start()

    def get(self) -> tuple:
        if self._thread is not None:
            self._thread.join()
            self._thread = None
        if self._exc is not None:
            exc, self._exc = self._exc, None
            raise exc
        caller = torch.cuda.current_stream(self._graph.device)
        caller.wait_stream(self._prefetch_stream)
        # the ring plan made by prepare() on the side stream is now ordered before
        # the caller's stream, where advance() commits it
        self._graph._adopt_plan(caller)
        result, self._result = self._result, None
        # the batch's tensors were allocated on the side stream and are used on
        # the caller's from here on: without this, memory the caller frees could be
        # reused by a later prefetch while the caller's queued work still reads it
        _record_stream(result, caller, set())
        return result

    def prepare(self, raw_batch: RawBatch) -> PreparedBatch:
        return self._pipeline.prepare(raw_batch)


def _record_stream(obj, stream, seen: set) -> None:
    """record_stream(stream) on every device tensor inside obj (tensors, lists,
    tuples, dicts and dataclass instances such as PreparedBatch / NeighborData)."""
    if obj is None or id(obj) in seen:
        return
    seen.add(id(obj))
    if isinstance(obj, torch.Tensor):
        if obj.is_cuda:
            obj.record_stream(stream)
    elif isinstance(obj, (list, tuple)):
        for x in obj:
            _record_stream(x, stream, seen)
    elif isinstance(obj, dict):
        for x in obj.values():
            _record_stream(x, stream, seen)
    elif dataclasses.is_dataclass(obj) and not isinstance(obj, type):
        for f in dataclasses.fields(obj):
            _record_stream(getattr(obj, f.name), stream, seen)
