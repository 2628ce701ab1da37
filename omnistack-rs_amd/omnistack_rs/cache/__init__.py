"""Page-granular compressed KV cache (the paged cache the reference plans
for its serving loop: MANIFEST.md:211-215, ``page_size`` in config.py:43)."""
from .paged import PagedKVAttention, PagedKVCache, paged_attention

__all__ = ["PagedKVAttention", "PagedKVCache", "paged_attention"]
