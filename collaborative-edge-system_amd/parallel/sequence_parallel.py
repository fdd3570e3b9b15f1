"""``collab_infer.parallel.sequence_parallel`` (collab_infer/parallel/sequence_parallel.py:
283-292): one rank's ring / Ulysses / distributed-KV share, with the collectives replaced by a
:class:`LocalGroup` of simulated ranks on one GPU."""

from ..sequence_parallel import (  # noqa: F401
    LocalGroup,
    distributed_kv_attention,
    gather_heads,
    gather_sequence,
    ring_attention,
    shard_sequence,
    ulysses_attention,
    ulysses_gather,
    ulysses_scatter,
)

__all__ = [
    "distributed_kv_attention",
    "gather_heads",
    "gather_sequence",
    "ring_attention",
    "shard_sequence",
    "ulysses_attention",
    "ulysses_gather",
    "ulysses_scatter",
]
