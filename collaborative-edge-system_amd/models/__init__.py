"""The import paths of ``collab_infer.models`` for this path's layer ops.

``<pkg>.models.llama`` exports the layer ops of collab_infer/models/llama.py (``RMSNorm``,
``RotaryEmbedding``, ``apply_rotary`` and the ``act(gate) * up`` gates of its activation
table) and ``<pkg>.models.cache`` the per-layer KV cache (collab_infer/models/cache.py).
The model definitions around them (``ParallelAttention``, ``ParallelMLP``, ``DecoderLayer``,
``LlamaStage``, weight loading) are outside this path and are not provided.
"""

from . import cache, llama  # noqa: F401
