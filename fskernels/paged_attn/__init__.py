"""Paged KV cache and paged decode (reference: fskernels/paged_attn/__init__.py:1-4)."""
from .paged_kv_cache import PAGE_SIZE, PagedKVCache
from ..hip.decode import paged_flash_decode

__all__ = ["PagedKVCache", "PAGE_SIZE", "paged_flash_decode"]
