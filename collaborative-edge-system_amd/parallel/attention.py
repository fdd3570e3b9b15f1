"""``collab_infer.parallel.attention`` (collab_infer/parallel/attention.py:304-315): attention
with LSE, plain attention, the exact merges and the masking / GQA helpers, computed by the
gfx950 kernels."""

from ..attention import (  # noqa: F401
    MASK_CHUNK_ELEMENTS,
    KVMap,
    accumulation_dtype,
    attention,
    attention_with_lse,
    expand_kv,
    fully_masked,
    gqa_group,
    merge_attention,
    merge_attention_list,
    visibility_mask,
)

__all__ = [
    "MASK_CHUNK_ELEMENTS",
    "accumulation_dtype",
    "attention",
    "attention_with_lse",
    "expand_kv",
    "fully_masked",
    "gqa_group",
    "merge_attention",
    "merge_attention_list",
    "visibility_mask",
]
