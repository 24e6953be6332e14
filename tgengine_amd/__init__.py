"""tgengine_amd -- MI355X-native fused temporal data pipeline.

Drop-in for tgengine's TemporalGraph / GatherSpec / NeighborSpec /
PreparedBatch / DataPipeline path; every device computation runs in the HIP
library libtgx.so (built by ``python -m tgengine_amd.build``).
"""
from .core import (GatherSpec, NeighborData, NeighborSpec, PreparedBatch, RawBatch, Snapshot,
                   TemporalDataset, TemporalGraph, load_dataset)
from .pipeline import AsyncDataPipeline, DataPipeline

__all__ = ["AsyncDataPipeline", "DataPipeline", "GatherSpec", "NeighborData", "NeighborSpec",
           "PreparedBatch", "RawBatch", "Snapshot", "TemporalDataset", "TemporalGraph",
           "load_dataset"]
