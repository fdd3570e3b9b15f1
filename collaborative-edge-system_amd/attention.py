"""Attention kernels returning the log-sum-exp (LSE), on MI355X.

Drop-in for ``collab_infer.parallel.attention`` (collab_infer/parallel/attention.py): same
function names, signatures, masking rule and ``(out, lse)`` convention.  The compute runs in
hand-written gfx950 kernels reached through the C ABI of ``include/collab_edge_attn.h``:

* bf16 / f16 inputs with head size 64 or 128: matrix-core (MFMA) prefill kernel;
* other head sizes, f32 and f64 inputs: the generic online-softmax kernel;
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
from ctypes import byref
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


def _launch(q, k, v, q_pos, k_pos, causal, scale, mapping, out, lse, accumulate: bool) -> None:
    """One kernel call of cea_attention_with_lse on the current stream."""
    lib = nat.load_library()
    dev = q.device
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    ws_bytes = lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, nat.DTYPE_CODES[q.dtype])
    ws = nat.workspace(ws_bytes, dev)
    km, kn = nat.kv_map_arg(mapping)
    args = [nat.tensor_arg(t) for t in (q, k, v, q_pos, k_pos)]
    o = nat.tensor_arg(out)
    l = nat.tensor_arg(lse) if lse is not None else None
    rc = lib.cea_attention_with_lse(
        *(byref(a) for a in args), int(bool(causal)), float(scale), km, kn,
        byref(o), byref(l) if l is not None else None, int(accumulate),
        ws.data_ptr(), ws.numel(), nat.stream_of(dev))
    nat.check(rc, "attention_with_lse")


def _prepare(q, k, v, q_pos, k_pos, kv_map):
    nat.require_device(q, k, v, q_pos, k_pos)
    mapping = _kv_map_list(kv_map)
    _check_heads(q.shape[2], k.shape[2], mapping)
    q, k, v = (_inner_contiguous(t) for t in (q, k, v))
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k and v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    return q, k, v, _positions(q_pos), _positions(k_pos), mapping


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
    q, k, v, q_pos, k_pos, mapping = _prepare(q, k, v, q_pos, k_pos, kv_map)
    B, Sq, Hq, D = q.shape
    out = torch.empty(B, Sq, Hq, D, dtype=acc, device=q.device)
    lse = torch.empty(B, Hq, Sq, dtype=acc, device=q.device)
    if kv_block is not None and kv_block < Sk:
        out.zero_()
        lse.fill_(float("-inf"))
        for start in range(0, Sk, kv_block):
            end = min(start + kv_block, Sk)
            _launch(q, k[:, start:end], v[:, start:end], q_pos, k_pos[:, start:end], causal,
                    scale, mapping, out, lse, True)
        return out, lse
    _launch(q, k, v, q_pos, k_pos, causal, scale, mapping, out, lse, False)
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
    q, k, v, q_pos, k_pos, mapping = _prepare(q, k, v, q_pos, k_pos, kv_map)
    acc = accumulation_dtype(q.dtype)
    if out.dtype != acc or lse.dtype != acc:
        raise ValueError(f"running (out, lse) must be {acc}")
    if final is None:
        _launch(q, k, v, q_pos, k_pos, causal, scale, mapping, out, lse, bool(accumulate))
        return
    nat.require_device(final)
    lib = nat.load_library()
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    ws = nat.workspace(lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D,
                                                         nat.DTYPE_CODES[q.dtype]), q.device)
    km, kn = nat.kv_map_arg(mapping)
    args = [nat.tensor_arg(t) for t in (q, k, v, q_pos, k_pos, out, lse, final)]
    rc = lib.cea_attention_merge_final(
        *(byref(a) for a in args[:5]), int(bool(causal)), float(scale), km, kn,
        *(byref(a) for a in args[5:]), ws.data_ptr(), ws.numel(), nat.stream_of(q.device))
    nat.check(rc, "attention_merge_final")


def merge_attention(
    out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Exactly combine attention over two disjoint key sets (attention.py:242-250)."""
    nat.require_device(out_a, lse_a, out_b, lse_b)
    lib = nat.load_library()
    out_a, out_b = _inner_contiguous(out_a), _inner_contiguous(out_b)
    out = torch.empty(out_a.shape, dtype=out_a.dtype, device=out_a.device)
    lse = torch.empty(lse_a.shape, dtype=lse_a.dtype, device=lse_a.device)
    a = [nat.tensor_arg(t) for t in (out_a, lse_a, out_b, lse_b, out, lse)]
    rc = lib.cea_merge_attention(*(byref(x) for x in a), nat.stream_of(out.device))
    nat.check(rc, "merge_attention")
    return out, lse


def _merge_list(outs, lses, out_dtype=None):
    lib = nat.load_library()
    outs = [_inner_contiguous(o) for o in outs]
    dev = outs[0].device
    out = torch.empty(outs[0].shape, dtype=out_dtype or outs[0].dtype, device=dev)
    lse = torch.empty(lses[0].shape, dtype=lses[0].dtype, device=dev)
    oa, la = nat.tensor_array(outs), nat.tensor_array(lses)
    o, l = nat.tensor_arg(out), nat.tensor_arg(lse)
    rc = lib.cea_merge_attention_list(len(outs), oa, la, byref(o), byref(l),
                                      nat.stream_of(dev))
    nat.check(rc, "merge_attention_list")
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
    nat.require_device(*outs, *lses)
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
    nat.require_device(out, lse, packed)
    B, Sq, H, D = out.shape
    if packed is None:
        packed = torch.empty(B, Sq, H, D + 1, dtype=out.dtype, device=out.device)
    out = _inner_contiguous(out)
    lib = nat.load_library()
    a = [nat.tensor_arg(t) for t in (out, lse, packed)]
    rc = lib.cea_pack_partial(*(byref(x) for x in a), nat.stream_of(out.device))
    nat.check(rc, "pack_partial")
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
    nat.require_device(*parts)
    parts = [_inner_contiguous(p) for p in parts]
    B, Sq, H, D1 = parts[0].shape
    dev = parts[0].device
    if len(parts) > nat.MAX_PARTS:  # merge is associative: reduce in groups, then repack
        groups = [merge_packed(parts[i : i + nat.MAX_PARTS], return_lse=True)
                  for i in range(0, len(parts), nat.MAX_PARTS)]
        parts = [pack_partial(o, l) for o, l in groups]
    out = torch.empty(B, Sq, H, D1 - 1, dtype=out_dtype or parts[0].dtype, device=dev)
    lse = torch.empty(B, H, Sq, dtype=parts[0].dtype, device=dev) if return_lse else None
    lib = nat.load_library()
    pa, oa = nat.tensor_array(parts), nat.tensor_arg(out)
    la = nat.tensor_arg(lse) if lse is not None else None
    rc = lib.cea_merge_packed(len(parts), pa, byref(oa), byref(la) if la is not None else None,
                              nat.stream_of(dev))
    nat.check(rc, "merge_packed")
    return (out, lse) if return_lse else out


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
    q, k, v, q_pos, k_pos, mapping = _prepare(q, k, v, q_pos, k_pos, kv_map)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _launch(q, k, v, q_pos, k_pos, causal, scale, mapping, out, None, False)
    return out


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
