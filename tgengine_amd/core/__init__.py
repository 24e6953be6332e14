"""Storage and kernels of the fused temporal data pipeline (reference tgengine/core)."""
from .batch import NeighborData, PreparedBatch, RawBatch
from .dataset import TemporalDataset, load_dataset
from .gather_spec import GatherSpec, NeighborSpec
from .temporal_graph import Snapshot, TemporalGraph

__all__ = ["GatherSpec", "NeighborData", "NeighborSpec", "PreparedBatch", "RawBatch",
           "Snapshot", "TemporalDataset", "TemporalGraph", "load_dataset"]
