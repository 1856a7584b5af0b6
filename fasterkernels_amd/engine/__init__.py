"""Model-level runner around the decode hot path (reference: fskernels/engine)."""
from .hip_graph_runner import HIPGraphCache, HIPGraphRunner, get_kv_from_hf_cache

__all__ = ["HIPGraphCache", "HIPGraphRunner", "get_kv_from_hf_cache"]
