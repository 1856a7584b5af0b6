"""HIP-graph decode steps and the whole-model graph runner (the reference's fskernels/engine)."""
from .hip_graph import DecodeGraph, PagedDecodeStep
from .hip_graph_runner import HIPGraphCache, HIPGraphRunner

__all__ = ["DecodeGraph", "PagedDecodeStep", "HIPGraphCache", "HIPGraphRunner"]
