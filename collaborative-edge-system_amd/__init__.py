"""MI355X (gfx950) implementation of collab_infer's per-device attention hot path.

Import with ``importlib.import_module("collaborative-edge-system_amd")``.  Modules:

* :mod:`.attention` - ``attention_with_lse``, ``attention``, ``merge_attention``,
  ``merge_attention_list`` and helpers (collab_infer/parallel/attention.py)
* :mod:`.sequence_parallel` - one rank's ring / Ulysses / distributed-KV share on one GPU
  (collab_infer/parallel/sequence_parallel.py)
* :mod:`.layers` - RMSNorm, rotary, SiLU-gate (collab_infer/models/llama.py)
* :mod:`.kv_cache` - head-major KV cache with the rotary of K fused into the append
  (collab_infer/models/cache.py)
* :mod:`.partition` - splits and sequence layouts (collab_infer/parallel/partition.py)
* :mod:`.projection` - the fused Q/K/V and gate/up projections (own gfx950 GEMM; column views,
  gate/up with the activation fused)
  (collab_infer/parallel/tensor_parallel.py:264-320)
* :mod:`.workloads` - seeded inputs of the five measured workloads
* :mod:`.parallel` / :mod:`.models` - the reference's import paths
  (``parallel.attention``, ``parallel.sequence_parallel``, ``parallel.partition``,
  ``models.llama``, ``models.cache``) with its public names and signatures
"""

from . import _native, attention, kv_cache, layers, partition, projection, sequence_parallel, workloads  # noqa: F401
from . import models, parallel  # noqa: F401
from .attention import (  # noqa: F401
    MASK_CHUNK_ELEMENTS,
    accumulation_dtype,
    attention as attention_fn,
    attention_with_lse,
    attention_with_lse_into,
    expand_kv,
    fully_masked,
    gqa_group,
    merge_attention,
    merge_attention_list,
    merge_packed,
    pack_partial,
    visibility_mask,
)
from .kv_cache import LayerKVCache, kv_append  # noqa: F401
from .layers import (  # noqa: F401
    RMSNorm,
    RotaryEmbedding,
    apply_rotary,
    gated_activation,
    gated_mul,
    rmsnorm,
    rmsnorm_rope,
    silu_mul,
)
from .partition import HeadShard, SequenceLayout, partition_heads, split_sizes  # noqa: F401
from .projection import FusedColumnParallelLinear, fused_linear, linear, linear_gated  # noqa: F401
from .sequence_parallel import (  # noqa: F401
    LocalGroup,
    distributed_kv_attention,
    distributed_kv_attention_packed,
    gather_heads,
    gather_sequence,
    partitioned_attention,
    ring_attention,
    ulysses_attention,
    ulysses_gather,
    ulysses_scatter,
)

__version__ = "0.1.0"
