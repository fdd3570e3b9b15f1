"""Attention kernels returning the log-sum-exp (LSE), on MI355X.

Drop-in for ``collab_infer.parallel.attention`` (collab_infer/parallel/attention.py): same
function names, signatures, masking rule and ``(out, lse)`` convention.  The compute runs in
hand-written gfx950 kernels, reached through the PyTorch operators ``torch.ops.collab_edge``
(a thin C++ layer that allocates outputs and calls the C ABI of
``include/collab_edge_attn.h`` on PyTorch's current stream):

* bf16 / f16 inputs with head size 64 or 128: matrix-core (MFMA) prefill kernel;
* f32 inputs with head size 64 or 128: the f32 matrix-core kernel;
* other head sizes and f64 inputs: the generic online-softmax kernel;
* merges: the HBM-bound exact LSE merge kernels.

Masking is defined by explicit token positions (attention.py:7-13)::

    key j is visible to query i  <=>  k_pos[j] >= 0  and  (not causal or k_pos[j] <= q_pos[i])

``q`` is ``[B, Sq, Hq, D]``, ``k``/``v`` are ``[B, Sk, Hkv, D]`` (any strides, the kernels
read head-major cache views in place), positions are ``[B, S]`` int64.  Rows with no
visible key give ``out = 0`` and ``lse = -inf``.  Masks are never materialised: the kernels
classify every 64-key tile from its position range and skip, run unmasked, or mask element
by element, without host synchronisation.
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple, Union

import torch

from . import _native as nat

KVMap = Optional[Union[torch.Tensor, Sequence[int]]]

# The reference bounds the memory of a materialised mask with this many elements per call
# (attention.py:39).  The kernels never build a mask; the constant is kept for callers.
MASK_CHUNK_ELEMENTS = 1 << 22


def accumulation_dtype(dtype: torch.dtype) -> torch.dtype:
    """f64 for f64 inputs, f32 otherwise (attention.py:56-57)."""
    return torch.float64 if dtype == torch.float64 else torch.float32


def _kv_map_list(kv_map: KVMap) -> Optional[List[int]]:
    if kv_map is None:
        return None
    if isinstance(kv_map, torch.Tensor):
        return [int(x) for x in kv_map.reshape(-1).tolist()]
    return [int(x) for x in kv_map]


def expand_kv(x: torch.Tensor, num_q_heads: int, kv_map: KVMap = None) -> torch.Tensor:
    """Repeat KV heads so head ``h`` of the result serves query head ``h`` (attention.py:68-82)."""
    mapping = _kv_map_list(kv_map)
    n_kv = x.shape[2]
    if mapping is None:
        if n_kv == num_q_heads:
            return x
        if num_q_heads % n_kv != 0:
            raise ValueError(f"{num_q_heads} query heads cannot share {n_kv} KV heads evenly")
        return x.repeat_interleave(num_q_heads // n_kv, dim=2)
    if len(mapping) != num_q_heads:
        raise ValueError("kv_map must have one entry per query head")
    if n_kv == num_q_heads and mapping == list(range(num_q_heads)):
        return x
    return x.index_select(2, torch.tensor(mapping, dtype=torch.long, device=x.device))


def gqa_group(num_q_heads: int, num_kv_heads: int, kv_map: KVMap = None) -> Optional[int]:
    """Group size ``g`` if query head ``h`` uses KV head ``h // g``, else ``None`` (attention.py:85-93)."""
    if num_kv_heads < 1 or num_q_heads % num_kv_heads:
        return None
    g = num_q_heads // num_kv_heads
    mapping = _kv_map_list(kv_map)
    if mapping is None:
        return g
    return g if mapping == [h // g for h in range(num_q_heads)] else None


def visibility_mask(q_pos: torch.Tensor, k_pos: torch.Tensor, causal: bool = True) -> torch.Tensor:
    """Boolean ``[B, 1, Sq, Sk]`` mask of visible (query, key) pairs (attention.py:96-101)."""
    vis = (k_pos >= 0)[:, None, None, :]
    if causal:
        vis = vis & (k_pos[:, None, None, :] <= q_pos[:, None, :, None])
    return vis.expand(q_pos.shape[0], 1, q_pos.shape[1], k_pos.shape[1])


def fully_masked(q_pos: torch.Tensor, k_pos: torch.Tensor, causal: bool = True) -> bool:
    """Whether no query can see any key (attention.py:104-113).  A host-side helper; the
    kernels make the same decision per 64-key tile on the device."""
    if k_pos.numel() == 0 or q_pos.numel() == 0:
        return True
    valid = k_pos[k_pos >= 0]
    if valid.numel() == 0:
        return True
    if not causal:
        return False
    return bool(q_pos.max() < valid.min())


def _empty_result(q: torch.Tensor, acc: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    B, Sq, Hq, D = q.shape
    return (
        torch.zeros(B, Sq, Hq, D, dtype=acc, device=q.device),
        torch.full((B, Hq, Sq), float("-inf"), dtype=acc, device=q.device),
    )


def _inner_contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dim() == 0 or t.shape[-1] <= 1 or t.stride(-1) == 1) else t.contiguous()


def _positions(p: torch.Tensor) -> torch.Tensor:
    return p if p.dtype == torch.int64 else p.to(torch.int64)


def _check_heads(num_q: int, num_kv: int, mapping: Optional[List[int]]) -> None:
    if mapping is None:
        if num_kv < 1 or num_q % num_kv:
            raise ValueError(f"{num_q} query heads cannot share {num_kv} KV heads evenly")
    elif len(mapping) != num_q:
        raise ValueError("kv_map must have one entry per query head")


def _prepare(q, k, v, kv_map):
    mapping = _kv_map_list(kv_map)
    _check_heads(q.shape[2], k.shape[2], mapping)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k and v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    return mapping


def attention_with_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos: torch.Tensor,
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    kv_block: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Masked softmax attention returning ``(out, lse)`` in accumulation precision
    (attention.py:201-239).

    ``out`` is ``[B, Sq, Hq, D]`` and ``lse`` is ``[B, Hq, Sq]`` (natural log).  Rows without
    any visible key produce ``out = 0`` and ``lse = -inf``.  ``kv_block`` processes the keys
    in blocks whose partial results are merged exactly, as the reference does.
    """
    acc = accumulation_dtype(q.dtype)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    Sk = k.shape[1]
    if Sk == 0 or q.shape[1] == 0:
        return _empty_result(q, acc)
    if kv_block is not None and kv_block < 1:
        # the reference's range(0, Sk, 0) raises; a negative block size is rejected too
        raise ValueError("kv_block must be positive")
    mapping = _prepare(q, k, v, kv_map)
    ops = nat.ops()
    if kv_block is not None and kv_block < Sk:
        out, lse = _empty_result(q, acc)
        for start in range(0, Sk, kv_block):
            end = min(start + kv_block, Sk)
            ops.attention_into(out, lse, q, k[:, start:end], v[:, start:end], q_pos,
                               k_pos[:, start:end], bool(causal), scale, mapping, True, None)
        return out, lse
    out, lse = ops.attention(q, k, v, q_pos, k_pos, bool(causal), scale, mapping, True)
    return out, lse


def attention_with_lse_into(
    out: torch.Tensor,
    lse: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos: torch.Tensor,
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    accumulate: bool = True,
    final: Optional[torch.Tensor] = None,
) -> None:
    """Merges attention over one more KV block into a running ``(out, lse)`` in place.

    Equivalent to ``out, lse = merge_attention(out, lse, *attention_with_lse(...))`` (the
    online merge of ring attention, sequence_parallel.py:117-121) without materialising the
    block's partial result: the merge runs in the attention kernel's epilogue.  Start from
    ``out = 0``, ``lse = -inf`` (the merge's neutral element), or pass
    ``accumulate=False`` for the first block: its result then overwrites ``(out, lse)``,
    which need no initialisation (an empty block leaves them untouched either way).

    ``final`` (``[B, Sq, Hq, D]`` in q's dtype or the accumulation dtype) receives the merged
    output instead of ``out`` - the last step of a ring with its ``out.to(q.dtype)``
    (sequence_parallel.py:121, 128) in the same kernel; ``out`` is then left unspecified.
    """
    if final is not None and not accumulate:
        raise ValueError("final needs accumulate=True")
    if q.shape[1] == 0 or (k.shape[1] == 0 and final is None):
        return
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    mapping = _prepare(q, k, v, kv_map)
    acc = accumulation_dtype(q.dtype)
    if out.dtype != acc or lse.dtype != acc:
        raise ValueError(f"running (out, lse) must be {acc}")
    nat.ops().attention_into(out, lse, q, k, v, q_pos, k_pos, bool(causal), scale, mapping,
                             bool(accumulate), final)


def merge_attention(
    out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Exactly combine attention over two disjoint key sets (attention.py:242-250)."""
    out, lse = nat.ops().merge([out_a, out_b], [lse_a, lse_b], True, None)
    return out, lse


def _merge_list(outs, lses, out_dtype=None):
    out, lse = nat.ops().merge(list(outs), list(lses), False, out_dtype)
    return out, lse


def merge_attention_list(
    outs: Sequence[torch.Tensor], lses: Sequence[torch.Tensor]
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Combine any number of partial attention results (attention.py:253-264)."""
    outs, lses = list(outs), list(lses)
    if len(outs) != len(lses) or not outs:
        raise ValueError("need the same positive number of outputs and lses")
    if len(outs) == 1:
        return outs[0], lses[0]
    while len(outs) > nat.MAX_PARTS:  # merge is associative: reduce in groups
        grouped = [
            _merge_list(outs[i : i + nat.MAX_PARTS], lses[i : i + nat.MAX_PARTS])
            for i in range(0, len(outs), nat.MAX_PARTS)
        ]
        outs = [o for o, _ in grouped]
        lses = [l for _, l in grouped]
        if len(outs) == 1:
            return outs[0], lses[0]
    return _merge_list(outs, lses)


def pack_partial(out: torch.Tensor, lse: torch.Tensor,
                 packed: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The all-gather message of distributed-KV decoding: ``[B, Sq, H, D+1]`` holding ``out``
    and, in the last slot, ``lse`` (sequence_parallel.py:275,
    ``torch.cat([o, l.transpose(1, 2).unsqueeze(-1)], dim=-1)``).  ``packed`` may be a slot
    of a preallocated gathered buffer ``[n, B, Sq, H, D+1]``."""
    if packed is None:
        B, Sq, H, D = out.shape
        packed = torch.empty(B, Sq, H, D + 1, dtype=out.dtype, device=out.device)
    nat.ops().pack_partial(out, lse, packed)
    return packed


def merge_packed(gathered, out_dtype: Optional[torch.dtype] = None, return_lse: bool = False):
    """Exact merge of all-gathered packed partials, read in place (sequence_parallel.py:277-280:
    ``outs = [p[..., :D]]``, ``lses = [p[..., D].transpose(1, 2)]``, ``merge_attention_list``
    and the cast to the query dtype).

    ``gathered`` is the ``[n, B, Sq, H, D+1]`` buffer or a sequence of ``[B, Sq, H, D+1]``
    parts; returns ``out`` in ``out_dtype`` (default the parts' dtype), plus the merged lse
    when ``return_lse``."""
    parts = list(gathered.unbind(0)) if isinstance(gathered, torch.Tensor) else list(gathered)
    if not parts:
        raise ValueError("need at least one packed partial")
    while len(parts) > nat.MAX_PARTS:  # merge is associative: reduce in groups, then repack
        groups = [merge_packed(parts[i : i + nat.MAX_PARTS], return_lse=True)
                  for i in range(0, len(parts), nat.MAX_PARTS)]
        parts = [pack_partial(o, l) for o, l in groups]
    res = nat.ops().merge_packed(parts, out_dtype or parts[0].dtype, bool(return_lse))
    return (res[0], res[1]) if return_lse else res[0]


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos: torch.Tensor,
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    kv_block: Optional[int] = None,
) -> torch.Tensor:
    """Single-device attention; returns ``[B, Sq, Hq, D]`` in ``q.dtype`` (attention.py:270-301)."""
    Sk = k.shape[1]
    if kv_block is not None and kv_block < Sk:
        out, _ = attention_with_lse(q, k, v, q_pos, k_pos, causal=causal, scale=scale,
                                    kv_map=kv_map, kv_block=kv_block)
        return out.to(q.dtype)
    if Sk == 0 or q.shape[1] == 0:
        return torch.zeros_like(q)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    mapping = _prepare(q, k, v, kv_map)
    return nat.ops().attention(q, k, v, q_pos, k_pos, bool(causal), scale, mapping, False)[0]


__all__ = [
    "MASK_CHUNK_ELEMENTS",
    "accumulation_dtype",
    "attention",
    "attention_with_lse",
    "attention_with_lse_into",
    "expand_kv",
    "fully_masked",
    "gqa_group",
    "merge_attention",
    "merge_attention_list",
    "merge_packed",
    "pack_partial",
    "visibility_mask",
]
