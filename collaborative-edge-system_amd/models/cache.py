"""``collab_infer.models.cache.LayerKVCache`` (collab_infer/models/cache.py:11-85): the
head-major per-layer KV cache, appended by the fused rotary + append kernel."""

from ..kv_cache import LayerKVCache, kv_append  # noqa: F401

__all__ = ["LayerKVCache"]
