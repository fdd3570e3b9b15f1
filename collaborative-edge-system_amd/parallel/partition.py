"""``collab_infer.parallel.partition`` (collab_infer/parallel/partition.py:247-254): weighted
splits, head shards and sequence layouts."""

from ..partition import (  # noqa: F401
    HeadShard,
    SequenceLayout,
    default_kv_map,
    offsets_of,
    partition_heads,
    split_sizes,
)

__all__ = [
    "HeadShard",
    "SequenceLayout",
    "default_kv_map",
    "offsets_of",
    "partition_heads",
    "split_sizes",
]
