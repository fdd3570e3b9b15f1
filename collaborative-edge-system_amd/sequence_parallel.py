"""One rank's share of ring attention, Ulysses attention and distributed-KV decoding, run on
one GPU.

Drop-in signatures of collab_infer/parallel/sequence_parallel.py.  This package runs no
collectives: the ``comm`` argument is a :class:`LocalGroup` that already holds what the other
simulated ranks would send (their KV blocks, partitions or token shards), so a rank's share
is computed at its real shape by streaming those blocks through the kernels:

* :func:`ring_attention` (sequence_parallel.py:68-130) - the rank's queries against every
  rank's KV block in ring order ``(r - step) mod n``, merged exactly: one
  ``cea_ring_attention`` call whose single prefill launch carries each query row's softmax
  state across the blocks, or, where one launch does not fit, block after block with each
  block merged into a running ``(out, lse)`` in the attention kernel's epilogue.  Fully
  hidden blocks cost one pass over their position summaries (the kernel skips their tiles),
  which replaces the reference's host-side ``fully_masked`` test without a device-to-host
  sync.
* :func:`distributed_kv_attention` (sequence_parallel.py:250-280) - a replicated query
  against every rank's cache partition, partials merged exactly (``merge_attention_list``).
* :func:`ulysses_scatter` / :func:`ulysses_gather` / :func:`ulysses_attention`
  (sequence_parallel.py:143-239) - the all-to-all data movement as concatenation, then the
  head-sharded local attention over the full sequence.

A group of size 1 is the single-device case of the reference (its ``n == 1`` branches).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _native as nat
from .attention import (
    KVMap,
    _kv_map_list,
    _check_heads,
    _inner_contiguous,
    _positions,
    accumulation_dtype,
    attention,
    attention_with_lse,
    attention_with_lse_into,
    _merge_list,
    merge_attention_list,
    merge_packed,
    pack_partial,
)
from .partition import HeadShard, SequenceLayout, offsets_of

import math


class LocalGroup:
    """A group of ``size`` simulated ranks on one GPU, seen from rank ``rank``.

    It stands in for collab_infer's ``Communicator`` (distributed/comm.py:200): instead of
    exchanging messages, every rank's shard is registered up front with :meth:`set_shard`
    (keys ``k``, ``v``, ``pos`` for KV blocks; ``q`` too for Ulysses).  ``wire_dtype`` is the
    communicator's activation wire dtype (``comm_dtype``, distributed/comm.py:259-262) with
    its rules (comm.py:275-290): a floating tensor travels in it only when it is narrower
    than the tensor's own dtype, and float16 saturates at +-65504 instead of overflowing.
    Pieces that cross the wire are rounded through it on arrival.
    """

    def __init__(self, size: int, rank: int = 0, wire_dtype: Optional[torch.dtype] = None) -> None:
        if size < 1 or not 0 <= rank < size:
            raise ValueError(f"invalid rank {rank} for a group of {size}")
        self.size = int(size)
        self.rank = int(rank)
        self.wire_dtype = wire_dtype
        self._shards: Dict[int, Dict[str, torch.Tensor]] = {}

    def set_shard(self, rank: int, **tensors: torch.Tensor) -> "LocalGroup":
        self._shards.setdefault(int(rank), {}).update(tensors)
        return self

    def shard(self, rank: int) -> Dict[str, torch.Tensor]:
        if rank not in self._shards:
            raise RuntimeError(f"no data registered for simulated rank {rank}")
        return self._shards[rank]

    def view_as(self, rank: int) -> "LocalGroup":
        """The same group seen from another rank (shares the registered shards)."""
        g = LocalGroup(self.size, rank, self.wire_dtype)
        g._shards = self._shards
        return g

    def wire_dtype_for(self, dtype: torch.dtype) -> torch.dtype:
        """The dtype ``dtype`` travels in (Communicator.wire_dtype, comm.py:284-290)."""
        wire = self.wire_dtype
        if wire is None or not dtype.is_floating_point:
            return dtype
        itemsize = torch.empty(0, dtype=dtype).element_size()
        return wire if torch.empty(0, dtype=wire).element_size() < itemsize else dtype

    def to_wire(self, t: torch.Tensor) -> torch.Tensor:
        """``t`` in its wire dtype (Communicator.to_wire, comm.py:275-282)."""
        wire = self.wire_dtype_for(t.dtype)
        if wire == t.dtype:
            return t
        if wire == torch.float16:
            t = t.clamp(-65504.0, 65504.0)
        return t.to(wire)

    def received(self, t: torch.Tensor) -> torch.Tensor:
        """``t`` as it arrives after a compressed transfer (sent in the wire dtype, cast back)."""
        w = self.to_wire(t)
        return t if w is t else w.to(t.dtype)

    def gathered(self, key: str, local: torch.Tensor, compress: bool = False) -> List[torch.Tensor]:
        """What a collective delivers to this rank, in rank order: its own tensor ``local``
        and every other rank's tensor registered under ``key``.  A compressed transfer sends
        every piece, the rank's own included, through the wire dtype (comm.py:484-486)."""
        out = [local if r == self.rank else self.shard(r)[key] for r in range(self.size)]
        return [self.received(t) for t in out] if compress else out


def _kv_from(comm: LocalGroup, src: int, own: Tuple[torch.Tensor, torch.Tensor, torch.Tensor]):
    """The KV block of rank ``src`` as the ring delivers it: received blocks went through
    the wire dtype (sequence_parallel.py:103, 127), the own block did not."""
    if src == comm.rank:
        return own
    s = comm.shard(src)
    return comm.received(s["k"]), comm.received(s["v"]), s["pos"]


def _raw_kv(comm: LocalGroup, src: int):
    """The KV partition rank ``src`` stores, untouched by any wire rounding."""
    s = comm.shard(src)
    return s["k"], s["v"], s["pos"]


# --------------------------------------------------------------------------------------
# ring attention
# --------------------------------------------------------------------------------------
def _ring_pieces(k, v, k_pos, comm: LocalGroup, kv_sizes: Sequence[int], kv_block: Optional[int]):
    """The KV pieces rank ``comm.rank`` attends to, in ring order: the block of rank
    ``(r - step) mod n`` at step ``step`` (sequence_parallel.py:107-127), as the ring delivers
    it, split into ``kv_block``-key pieces when ``kv_block`` is given (attention.py:225-236)."""
    n, r = comm.size, comm.rank
    if kv_block is not None and kv_block < 1:
        raise ValueError("kv_block must be positive")
    if len(kv_sizes) != n or kv_sizes[r] != k.shape[1]:
        raise ValueError(f"kv_sizes {list(kv_sizes)} inconsistent with local block of {k.shape[1]} tokens")
    own = (k, v, k_pos)
    pieces = []
    for step in range(n):
        src = (r - step) % n
        kb, vb, pb = _kv_from(comm, src, own)
        if kb.shape[1] != kv_sizes[src]:
            raise ValueError(f"kv_sizes {list(kv_sizes)} inconsistent with the block of rank {src}")
        size = kb.shape[1]
        blk = kv_block if kv_block is not None and kv_block < size else max(size, 1)
        for start in range(0, size, blk):
            end = min(start + blk, size)
            pieces.append((kb[:, start:end], vb[:, start:end], pb[:, start:end]))
    return pieces


def _ring(q, k, v, q_pos, k_pos, comm, kv_sizes, causal, scale, kv_map, kv_block, with_lse):
    pieces = _ring_pieces(k, v, k_pos, comm, kv_sizes, kv_block)
    acc = accumulation_dtype(q.dtype)
    if not pieces:  # no rank held a key: the merge's neutral element
        out = torch.zeros(q.shape, dtype=acc if with_lse else q.dtype, device=q.device)
        lse = torch.full((q.shape[0], q.shape[2], q.shape[1]), float("-inf"), dtype=acc,
                         device=q.device)
        return (out, lse) if with_lse else out
    mapping = _kv_map_list(kv_map)
    for kb, vb, _ in pieces:
        _check_heads(q.shape[2], kb.shape[2], mapping)
        if kb.dtype != q.dtype or vb.dtype != q.dtype:
            raise ValueError(f"q, k and v must share a dtype, got {q.dtype}, {kb.dtype}, {vb.dtype}")
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    if len(pieces) <= nat.MAX_PARTS:
        # every piece in one call (cea_ring_attention): one launch for the MFMA kernel
        res = nat.ops().ring(q, q_pos, [x[0] for x in pieces], [x[1] for x in pieces],
                             [x[2] for x in pieces], bool(causal), scale, mapping, bool(with_lse))
        return (res[0], res[1]) if with_lse else res[0]
    # more pieces than one call takes: piece after piece, merged in the kernel epilogue
    B, Sq, Hq, D = q.shape
    out = torch.empty(B, Sq, Hq, D, dtype=acc, device=q.device)
    lse = torch.empty((B, Hq, Sq), dtype=acc, device=q.device)
    final = None if with_lse else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    for i, (kb, vb, pb) in enumerate(pieces):
        last = i == len(pieces) - 1
        attention_with_lse_into(out, lse, q, kb, vb, q_pos, pb, causal=causal, scale=scale,
                                kv_map=kv_map, accumulate=i > 0, final=final if last else None)
    return (out, lse) if with_lse else final


def ring_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos: torch.Tensor,
    comm: LocalGroup,
    kv_sizes: Sequence[int],
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    kv_block: Optional[int] = None,
) -> torch.Tensor:
    """Attention of this rank's queries over the KV blocks of all ranks
    (sequence_parallel.py:68-130); returns ``[B, s_r, Hq, D]`` in ``q.dtype``.

    Every block is resident here, so the rank's whole share is one call: its blocks in ring
    order form one kernel launch that carries each query row's softmax state from block to
    block and writes the result in ``q.dtype`` once (the reference's per-step merge and final
    ``out.to(q.dtype)``, :121 and :128).  Blocks no query can see cost one pass over their
    position summaries, which replaces the reference's ``fully_masked`` skip (:117)."""
    if comm.size == 1:
        out, _ = attention_with_lse(q, k, v, q_pos, k_pos, causal=causal, scale=scale,
                                    kv_map=kv_map, kv_block=kv_block)
        return out.to(q.dtype)
    return _ring(q, k, v, q_pos, k_pos, comm, kv_sizes, causal, scale, kv_map, kv_block, False)


def ring_attention_with_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos: torch.Tensor,
    comm: LocalGroup,
    kv_sizes: Sequence[int],
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    kv_block: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """:func:`ring_attention` returning the merged ``(out, lse)`` in accumulation precision."""
    if comm.size == 1:
        return attention_with_lse(q, k, v, q_pos, k_pos, causal=causal, scale=scale,
                                  kv_map=kv_map, kv_block=kv_block)
    return _ring(q, k, v, q_pos, k_pos, comm, kv_sizes, causal, scale, kv_map, kv_block, True)


# --------------------------------------------------------------------------------------
# distributed-KV decoding
# --------------------------------------------------------------------------------------
def partitioned_attention(
    q: torch.Tensor,
    q_pos: torch.Tensor,
    parts: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    out_dtype: Optional[torch.dtype] = None,
    return_lse: bool = False,
    return_parts: bool = False,
):
    """Attention of ``q`` against KV partitions ``[(k_p, v_p, pos_p), ...]`` plus the exact
    merge, in the kernels of ``cea_partitioned_attention``.

    Returns ``out`` (``out_dtype``, default ``q.dtype``), plus ``lse`` and the list of
    per-partition ``(out_p, lse_p)`` (each rank's ``attention_with_lse``) when asked.
    """
    parts = list(parts)
    if not parts:
        raise ValueError("need at least one partition")
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    mapping = _kv_map_list(kv_map)
    for p in parts:
        _check_heads(q.shape[2], p[0].shape[2], mapping)
    acc = accumulation_dtype(q.dtype)
    if out_dtype is None:  # the merged lse comes with an accumulation-precision output
        out_dtype = acc if return_lse else q.dtype
    if len(parts) > nat.MAX_PARTS:
        # more partitions than one launch takes: groups of up to MAX_PARTS, each one split-KV
        # launch with its reduction, then the exact merge of the groups (the merge is
        # associative; the reference merges all partials at once, attention.py:253-264)
        groups = [partitioned_attention(q, q_pos, parts[i:i + nat.MAX_PARTS], causal=causal,
                                        scale=scale, kv_map=mapping, out_dtype=acc,
                                        return_lse=True, return_parts=return_parts)
                  for i in range(0, len(parts), nat.MAX_PARTS)]
        out, lse = merge_attention_list([g[0] for g in groups], [g[1] for g in groups])
        result = [out.to(out_dtype)]
        if return_lse:
            result.append(lse)
        if return_parts:
            result.append([pr for g in groups for pr in g[2]])
        return result[0] if len(result) == 1 else tuple(result)
    res = nat.ops().partitioned(q, q_pos, [p[0] for p in parts], [p[1] for p in parts],
                                [p[2] for p in parts], bool(causal), scale, mapping, out_dtype,
                                bool(return_lse), bool(return_parts))
    out = res[0]
    lse = res[1] if return_lse else None
    rest = res[2 if return_lse else 1:]
    part_out, part_lse = rest[0::2], rest[1::2]
    result = [out]
    if return_lse:
        result.append(lse)
    if return_parts:
        result.append(list(zip(part_out, part_lse)))
    return result[0] if len(result) == 1 else tuple(result)


def _dkv_partitions(comm: LocalGroup, own):
    """Every rank's KV partition in rank order (the all-gather order).  Each rank attends to
    the partition it stores at full precision; only the f32 (out | lse) message crosses the
    wire, uncompressed (sequence_parallel.py:270-279)."""
    return [own if i == comm.rank else _raw_kv(comm, i) for i in range(comm.size)]


def distributed_kv_attention(
    q: torch.Tensor,
    k_local: torch.Tensor,
    v_local: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos_local: torch.Tensor,
    comm: LocalGroup,
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    kv_block: Optional[int] = None,
) -> torch.Tensor:
    """A replicated query against a KV cache sharded over the ranks of ``comm``
    (sequence_parallel.py:250-280); returns ``[B, Sq, Hq, D]`` in ``q.dtype``.

    Every rank's partition runs in one split-KV launch, the exact merge in its reduction;
    :func:`distributed_kv_attention_packed` runs the multi-device message flow instead."""
    if comm.size == 1:
        o, _ = attention_with_lse(q, k_local, v_local, q_pos, k_pos_local, causal=causal,
                                  scale=scale, kv_map=kv_map, kv_block=kv_block)
        return o.to(q.dtype)
    parts = _dkv_partitions(comm, (k_local, v_local, k_pos_local))
    if kv_block is not None:
        partial = [attention_with_lse(q, kk, vv, q_pos, pp, causal=causal, scale=scale,
                                      kv_map=kv_map, kv_block=kv_block) for kk, vv, pp in parts]
        o, _ = merge_attention_list([p[0] for p in partial], [p[1] for p in partial])
        return o.to(q.dtype)
    return partitioned_attention(q, q_pos, parts, causal=causal, scale=scale, kv_map=kv_map)


def distributed_kv_attention_packed(
    q: torch.Tensor,
    k_local: torch.Tensor,
    v_local: torch.Tensor,
    q_pos: torch.Tensor,
    k_pos_local: torch.Tensor,
    comm: LocalGroup,
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    kv_map: KVMap = None,
    kv_block: Optional[int] = None,
) -> torch.Tensor:
    """:func:`distributed_kv_attention` through the data flow of the multi-device version:
    each rank's partial ``(out, lse)`` is packed into its slot of the all-gathered
    ``[n, B, Sq, H, D+1]`` buffer (the message layout of sequence_parallel.py:275-276) and
    the buffer is merged in place, cast to ``q.dtype`` (:277-280)."""
    parts = _dkv_partitions(comm, (k_local, v_local, k_pos_local))
    B, Sq, Hq, D = q.shape
    gathered = torch.empty(comm.size, B, Sq, Hq, D + 1, dtype=accumulation_dtype(q.dtype),
                           device=q.device)
    for i, (kk, vv, pp) in enumerate(parts):
        o, l = attention_with_lse(q, kk, vv, q_pos, pp, causal=causal, scale=scale,
                                  kv_map=kv_map, kv_block=kv_block)
        pack_partial(o, l, gathered[i])
    return merge_packed(gathered, out_dtype=q.dtype)


# --------------------------------------------------------------------------------------
# Ulysses
# --------------------------------------------------------------------------------------
def _check_ulysses(comm: LocalGroup, seq_sizes: Sequence[int], head_shards: Sequence[HeadShard],
                   s_local: int) -> None:
    if len(seq_sizes) != comm.size or seq_sizes[comm.rank] != s_local:
        raise ValueError(f"seq_sizes {list(seq_sizes)} inconsistent with local shard of {s_local} tokens")
    if len(head_shards) != comm.size:
        raise ValueError("need one head shard per rank")


def _heads_contiguous(t: torch.Tensor) -> torch.Tensor:
    """``t`` with the heads of a token adjacent in memory (the copy kernels move whole token
    rows); a copy only for views that break this."""
    if t.shape[2] > 1 and t.stride(2) != t.shape[3] or t.stride(3) != 1 and t.shape[3] > 1:
        return t.contiguous()
    return t


def ulysses_scatter(q, k, v, positions, comm: LocalGroup, seq_sizes: Sequence[int],
                    head_shards: Sequence[HeadShard]):
    """Sequence-sharded -> head-sharded (sequence_parallel.py:143-179): this rank's heads over
    the whole sequence, tokens concatenated in rank order, with their positions ``[B, S]``.

    Every rank's shard is read where it lies and packed by one kernel
    (``cea_ulysses_scatter``) into this rank's receive buffer ``[B, S, q+2kv heads, D]``;
    ``q_f``, ``k_f``, ``v_f`` are head slices of it, as the reference's ``split`` returns.
    With wire compression every piece travels rounded through the wire dtype, as
    ``all_to_all(..., compress=True)`` does (distributed/comm.py:468-486)."""
    n, r = comm.size, comm.rank
    _check_ulysses(comm, seq_sizes, head_shards, q.shape[1])
    me = head_shards[r]
    shards = []
    for j in range(n):
        if j == r:
            sq, sk, sv, sp = q, k, v, positions
        else:
            s = comm.shard(j)
            sq, sk, sv, sp = s["q"], s["k"], s["v"], s["pos"]
            if sq.shape[1] != seq_sizes[j]:
                raise ValueError(f"seq_sizes {list(seq_sizes)} inconsistent with rank {j}")
        if n > 1:
            sq, sk, sv = (comm.received(x) for x in (sq, sk, sv))
        shards.append((_heads_contiguous(sq), _heads_contiguous(sk), _heads_contiguous(sv),
                       _positions(sp)))
    full, pos_f = nat.ops().ulysses_scatter([sh[0] for sh in shards], [sh[1] for sh in shards],
                                            [sh[2] for sh in shards], [sh[3] for sh in shards],
                                            me.q_start, me.q_count, me.kv_start, me.kv_count)
    q_f, k_f, v_f = full.split([me.q_count, me.kv_count, me.kv_count], dim=2)
    return q_f, k_f, v_f, pos_f


def _head_concat(outs: Sequence[torch.Tensor], start: int, length: int) -> torch.Tensor:
    """Tokens ``[start, start + length)`` of every part ``[B, S, h_j, D]``, heads
    concatenated in part order, by one kernel (``cea_ulysses_gather``)."""
    return nat.ops().ulysses_gather([_heads_contiguous(o) for o in outs], int(start), int(length))


def ulysses_gather(out_heads: torch.Tensor, comm: LocalGroup, seq_sizes: Sequence[int],
                   head_shards: Sequence[HeadShard]) -> torch.Tensor:
    """Second Ulysses all-to-all: head-sharded ``[B, S, h_r, D]`` -> ``[B, s_r, H, D]``
    (sequence_parallel.py:182-194).

    ``out_heads`` is this rank's head output over the whole sequence; the other simulated
    ranks' head outputs are read where they are registered in ``comm`` (``out_heads`` of
    each rank's shard), rounded through the wire dtype as the compressed all-to-all does.
    One kernel writes this rank's tokens with all heads."""
    n, r = comm.size, comm.rank
    if len(seq_sizes) != n:
        raise ValueError(f"seq_sizes {list(seq_sizes)} do not match a group of {n}")
    if len(head_shards) != n:
        raise ValueError("need one head shard per rank")
    outs = comm.gathered("out_heads", out_heads, compress=n > 1)
    for j, o in enumerate(outs):
        if o.shape[2] != head_shards[j].q_count:
            raise ValueError(f"rank {j} sent {o.shape[2]} heads, its shard has {head_shards[j].q_count}")
    return _head_concat(outs, offsets_of(seq_sizes)[r], seq_sizes[r])


def gather_heads(out_local: torch.Tensor, comm: LocalGroup,
                 head_shards: Sequence[HeadShard]) -> torch.Tensor:
    """All-gather of per-rank head slices ``[B, S, h_r, D]`` into ``[B, S, H, D]``
    (sequence_parallel.py:242-247, uncompressed): the other simulated ranks' slices are read
    where they are registered in ``comm`` (``out_heads``), and one kernel concatenates the
    heads in rank order."""
    if len(head_shards) != comm.size:
        raise ValueError("need one head shard per rank")
    if comm.size == 1:
        return out_local
    outs = comm.gathered("out_heads", out_local)
    S = out_local.shape[1]
    for j, o in enumerate(outs):
        if o.shape[2] != head_shards[j].q_count or o.shape[1] != S:
            raise ValueError(f"rank {j}'s slice {tuple(o.shape)} does not match its head shard")
    return _head_concat(outs, 0, S)


def ulysses_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    comm: LocalGroup,
    seq_sizes: Sequence[int],
    head_shards: Sequence[HeadShard],
    *,
    causal: bool = True,
    scale: Optional[float] = None,
    past: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
    kv_block: Optional[int] = None,
):
    """All-to-all sequence-parallel attention (sequence_parallel.py:197-239).

    Every simulated rank's head-sharded local attention runs here (the gather needs all of
    them); returns ``(out [B, s_r, Hq, D], (k_heads, v_heads, pos_full))`` for this rank.
    """
    out_mine = None
    mine = None
    for j in range(comm.size):
        cj = comm.view_as(j)
        if j == comm.rank:
            sq, sk, sv, sp = q, k, v, positions
        else:
            s = comm.shard(j)
            sq, sk, sv, sp = s["q"], s["k"], s["v"], s["pos"]
        q_f, k_f, v_f, pos_f = ulysses_scatter(sq, sk, sv, sp, cj, seq_sizes, head_shards)
        k_att, v_att, p_att = k_f, v_f, pos_f
        if j == comm.rank and past is not None and past[0].shape[1] > 0:
            k_att = torch.cat([past[0], k_f], dim=1)
            v_att = torch.cat([past[1], v_f], dim=1)
            p_att = torch.cat([past[2], pos_f], dim=1)
        elif j != comm.rank and "past" in comm.shard(j) and comm.shard(j)["past"][0].shape[1] > 0:
            pk, pv, pp = comm.shard(j)["past"]
            k_att, v_att, p_att = (torch.cat([pk, k_f], 1), torch.cat([pv, v_f], 1),
                                   torch.cat([pp, pos_f], 1))
        o = attention(q_f, k_att, v_att, pos_f, p_att, causal=causal, scale=scale,
                      kv_map=head_shards[j].kv_map, kv_block=kv_block)
        if j == comm.rank:
            out_mine = o
            mine = (k_f.contiguous(), v_f.contiguous(), pos_f)
        else:  # what rank j sends back in the second all-to-all
            comm.set_shard(j, out_heads=o)
    return ulysses_gather(out_mine, comm, seq_sizes, head_shards), mine


def gather_sequence(x_local: torch.Tensor, layout: SequenceLayout, comm: LocalGroup,
                    dim: int = 1) -> torch.Tensor:
    """All-gather sequence shards and restore global token order (sequence_parallel.py:55-62).
    The other simulated ranks' shards are read where they are registered in ``comm``
    (``x`` of each rank's shard)."""
    if comm.size == 1:
        return x_local
    return layout.unshard(comm.gathered("x", x_local), dim=dim)


def shard_sequence(x: torch.Tensor, layout: SequenceLayout, rank: int, dim: int = 1) -> torch.Tensor:
    """This rank's tokens of a full-sequence tensor (sequence_parallel.py:50-52)."""
    return layout.shard(x, rank, dim)


__all__ = [
    "LocalGroup",
    "distributed_kv_attention",
    "distributed_kv_attention_packed",
    "gather_heads",
    "gather_sequence",
    "partitioned_attention",
    "ring_attention",
    "ring_attention_with_lse",
    "shard_sequence",
    "ulysses_attention",
    "ulysses_gather",
    "ulysses_scatter",
]
