"""Who owns which tokens and heads: the host-side index arithmetic behind every rank's share.

Drop-in for collab_infer/parallel/partition.py (names, arguments, results and error types):

* :func:`split_sizes` - weighted integer split (partition.py:20-68).  The apportionment is
  Hamilton's largest-remainder method; its floating-point steps decide ties, so they are the
  reference's: share ``spare * w_i / sum(w)``, floor with a ``1e-9`` guard (plain floors if
  the guard over-assigns), leftover units to the largest fractional parts, lower index first.
* :class:`HeadShard` / :func:`partition_heads` - query heads and the KV heads they read
  (partition.py:83-160).  Heads are dealt out in units: whole KV groups when the grouping is
  regular and every rank can get one, single query heads otherwise.
* :class:`SequenceLayout` - contiguous or zigzag token ownership (partition.py:166-244),
  held as one table of chunks in global order; lookups bisect it and reassembly writes each
  chunk to its place.

Every rank of a deployment evaluates these functions identically, so ownership needs no
messages; on one GPU they decide which blocks a simulated rank streams.
"""

from __future__ import annotations

from dataclasses import dataclass

import bisect
import heapq
import itertools
import math
from typing import List, NamedTuple, Optional, Sequence, Tuple, Union

import torch

WeightsLike = Union[int, Sequence[float]]


# --------------------------------------------------------------------------------------
# weighted splits
# --------------------------------------------------------------------------------------
def _as_weights(weights: WeightsLike) -> List[float]:
    if isinstance(weights, int):
        if weights < 1:
            raise ValueError("number of parts must be >= 1")
        return [1.0] * weights
    w = [float(x) for x in weights]
    if not w:
        raise ValueError("weights must not be empty")
    bad = [x for x in w if not (math.isfinite(x) and x > 0)]
    if bad:
        raise ValueError(f"weights must be positive and finite, got {w}")
    return w


def _apportion(units: int, w: Sequence[float]) -> List[int]:
    """Hamilton's method: ``units`` integers proportional to ``w``, summing to ``units``."""
    total_w = sum(w)
    exact = [units * x / total_w for x in w]
    # a share that is an integer up to rounding error must not floor one below it; if the
    # guard hands out more than there is, fall back to plain floors
    got = [math.floor(e + 1e-9) for e in exact]
    if sum(got) > units:
        got = [math.floor(e) for e in exact]
    # the units still free go to the largest fractional parts, lower index first on ties
    winners = heapq.nsmallest(units - sum(got), range(len(w)), key=lambda i: (got[i] - exact[i], i))
    for i in winners:
        got[i] += 1
    return got


def split_sizes(total: int, weights: WeightsLike, granularity: int = 1, min_units: int = 1) -> List[int]:
    """Split ``total`` into parts proportional to ``weights`` (partition.py:20-68).

    Every part is a multiple of ``granularity`` holding at least ``min_units`` granules; the
    granules beyond those minimums are apportioned by :func:`_apportion`.
    """
    w = _as_weights(weights)
    if granularity < 1:
        raise ValueError("granularity must be >= 1")
    if total < 0 or total % granularity:
        raise ValueError(f"total={total} is not a non-negative multiple of granularity={granularity}")
    units, floor_units = total // granularity, len(w) * min_units
    if units < floor_units:
        raise ValueError(
            f"cannot split {total} (granularity {granularity}) into {len(w)} parts "
            f"with at least {min_units} unit(s) each"
        )
    return [(min_units + extra) * granularity for extra in _apportion(units - floor_units, w)]


def offsets_of(sizes: Sequence[int]) -> List[int]:
    """Start offset of every part (exclusive prefix sum)."""
    sizes = [int(s) for s in sizes]
    return list(itertools.accumulate(sizes[:-1], initial=0)) if sizes else []


# --------------------------------------------------------------------------------------
# attention heads
# --------------------------------------------------------------------------------------
@dataclass(frozen=True)
class HeadShard:
    """Query heads ``[q_start, q_start + q_count)`` of one rank and the KV heads
    ``[kv_start, kv_start + kv_count)`` they read (partition.py:83-105).  ``kv_map[i]`` is the
    shard-local KV head of the ``i``-th local query head; a KV head needed by several ranks
    appears in each of their shards.  A frozen dataclass with the reference's fields, so
    ``dataclasses.fields`` / ``replace`` / ``asdict`` and equality behave as there."""

    q_start: int
    q_count: int
    kv_start: int
    kv_count: int
    kv_map: Tuple[int, ...]

    @property
    def q_range(self) -> Tuple[int, int]:
        return self.q_start, self.q_start + self.q_count

    @property
    def kv_range(self) -> Tuple[int, int]:
        return self.kv_start, self.kv_start + self.kv_count


def default_kv_map(num_q_heads: int, num_kv_heads: int) -> List[int]:
    """Query head ``h`` reads KV head ``h // (num_q_heads / num_kv_heads)`` (partition.py:108-114)."""
    if num_kv_heads < 1 or num_q_heads % num_kv_heads:
        raise ValueError(f"num_q_heads={num_q_heads} must be a multiple of num_kv_heads={num_kv_heads}")
    per = num_q_heads // num_kv_heads
    return [h // per for h in range(num_q_heads)]


def _checked_map(num_q_heads: int, num_kv_heads: int, kv_map: Optional[Sequence[int]]) -> List[int]:
    table = default_kv_map(num_q_heads, num_kv_heads) if kv_map is None else [int(x) for x in kv_map]
    if len(table) != num_q_heads:
        raise ValueError("kv_map must have one entry per query head")
    if any(nxt < cur for cur, nxt in zip(table, table[1:])):
        raise ValueError("kv_map must be non-decreasing")
    if table and not (0 <= table[0] and table[-1] < num_kv_heads):
        raise ValueError("kv_map entries out of range")
    return table


def _group_width(num_q_heads: int, num_kv_heads: int, table: List[int]) -> int:
    """Query heads per KV head when the map is the regular ``h // g`` grouping, else 0."""
    if num_kv_heads < 1 or num_q_heads % num_kv_heads:
        return 0
    g = num_q_heads // num_kv_heads
    return g if all(kv == h // g for h, kv in enumerate(table)) else 0


def partition_heads(num_q_heads: int, num_kv_heads: int, weights: WeightsLike,
                    kv_map: Optional[Sequence[int]] = None) -> List[HeadShard]:
    """Deal the query heads, and the KV heads they read, out to ranks (partition.py:117-160).

    The dealing unit is a whole KV group when the map is regular and there are at least as
    many KV heads as ranks (no KV head is then held twice); otherwise single query heads,
    each rank holding every KV head its query heads read (MQA, or fewer KV heads than ranks).
    """
    table = _checked_map(num_q_heads, num_kv_heads, kv_map)
    ranks = weights if isinstance(weights, int) else len(weights)
    width = _group_width(num_q_heads, num_kv_heads, table)
    if width and num_kv_heads >= ranks:
        unit, n_units = width, num_kv_heads
    else:
        if num_q_heads < ranks:
            raise ValueError(f"cannot split {num_q_heads} query heads over {ranks} ranks")
        unit, n_units = 1, num_q_heads
    cuts = list(itertools.accumulate((unit * c for c in split_sizes(n_units, weights)), initial=0))
    shards = []
    for lo, hi in zip(cuts, cuts[1:]):
        used = table[lo:hi]
        base = used[0]
        shards.append(HeadShard(lo, hi - lo, base, used[-1] + 1 - base, tuple(t - base for t in used)))
    return shards


# --------------------------------------------------------------------------------------
# sequence layouts
# --------------------------------------------------------------------------------------
class _Chunk(NamedTuple):
    start: int    # global index of the chunk's first token
    length: int
    rank: int     # owner
    local: int    # offset of the chunk inside the owner's shard


class SequenceLayout:
    """Assignment of the tokens of a sequence to sequence-parallel ranks (partition.py:166-244).

    * ``contiguous``: rank ``r`` owns one run of consecutive tokens;
    * ``zigzag``: the sequence is cut into ``2n`` chunks, in global order the first halves of
      ranks ``0 .. n-1`` and then the second halves of ranks ``n-1 .. 0``; rank ``r`` owns its
      two halves (the first half of its ``sizes[r]`` tokens rounded down), which balances the
      causal work of ring attention.

    The layout is one table of non-empty chunks ``(start, length, rank, local offset)`` sorted
    by global start; ``segments[r]`` lists rank ``r``'s ``(start, length)`` in local order.
    """

    _KINDS = ("contiguous", "zigzag")

    def __init__(self, seq_len: int, num_ranks: int, weights: Optional[Sequence[float]] = None,
                 kind: str = "contiguous") -> None:
        if kind not in self._KINDS:
            raise ValueError(f"unknown sequence layout {kind!r}")
        self.seq_len = int(seq_len)
        self.num_ranks = int(num_ranks)
        self.kind = kind
        self.sizes = split_sizes(self.seq_len, list(weights) if weights else self.num_ranks)
        if len(self.sizes) != self.num_ranks:
            raise ValueError(f"{len(self.sizes)} weights for {self.num_ranks} ranks")
        n = self.num_ranks
        if kind == "contiguous":
            pieces = [(r, self.sizes[r], 0) for r in range(n)]
        else:
            lead = [s // 2 for s in self.sizes]
            pieces = [(r, lead[r], 0) for r in range(n)]
            pieces += [(r, self.sizes[r] - lead[r], lead[r]) for r in reversed(range(n))]
        starts = itertools.accumulate((length for _, length, _ in pieces), initial=0)
        self._chunks = [_Chunk(g0, length, r, loc) for g0, (r, length, loc) in zip(starts, pieces)
                        if length > 0]
        self._starts = [c.start for c in self._chunks]
        by_rank: List[List[_Chunk]] = [[] for _ in range(n)]
        for c in self._chunks:
            by_rank[c.rank].append(c)
        self._rank_chunks = [sorted(cs, key=lambda c: c.local) for cs in by_rank]
        self.segments = [[(c.start, c.length) for c in cs] for cs in self._rank_chunks]

    def local_len(self, rank: int) -> int:
        return self.sizes[rank]

    def indices(self, rank: int) -> torch.Tensor:
        """Global indices of the tokens of ``rank``, in local order."""
        runs = [torch.arange(c.start, c.start + c.length) for c in self._rank_chunks[rank]]
        return torch.cat(runs) if runs else torch.zeros(0, dtype=torch.long)

    def owner_of(self, index: int) -> Tuple[int, int]:
        """``(rank, local index)`` of global token ``index`` (negative counts from the end)."""
        g = index + self.seq_len if index < 0 else index
        if not 0 <= g < self.seq_len:
            raise IndexError(f"token index {index} out of range for length {self.seq_len}")
        c = self._chunks[bisect.bisect_right(self._starts, g) - 1]
        return c.rank, c.local + (g - c.start)

    def shard(self, x: torch.Tensor, rank: int, dim: int = 1) -> torch.Tensor:
        """The tokens of ``rank`` from a full-sequence tensor (a view when they are one run)."""
        runs = [x.narrow(dim, c.start, c.length) for c in self._rank_chunks[rank]]
        if len(runs) == 1:
            return runs[0]
        if not runs:
            return x.narrow(dim, 0, 0)
        return torch.cat(runs, dim=dim)

    def unshard(self, parts: Sequence[torch.Tensor], dim: int = 1) -> torch.Tensor:
        """Inverse of :meth:`shard`: every chunk of every rank's part written to its global place."""
        parts = list(parts)
        if len(parts) != self.num_ranks:
            raise ValueError(f"need {self.num_ranks} parts, got {len(parts)}")
        for r, p in enumerate(parts):
            if p.shape[dim] != self.sizes[r]:
                raise ValueError(f"part {r} holds {p.shape[dim]} tokens, the layout gives it {self.sizes[r]}")
        # what the reference's torch.cat of the pieces does: the other dimensions and the
        # device must agree (RuntimeError otherwise), mixed dtypes promote
        ref = parts[0]
        d = dim % ref.dim() if ref.dim() else dim
        dtype = ref.dtype
        for r, p in enumerate(parts[1:], 1):
            if p.dim() != ref.dim() or any(a != b for i, (a, b) in enumerate(zip(p.shape, ref.shape)) if i != d):
                raise RuntimeError(f"part {r} has shape {tuple(p.shape)}, part 0 {tuple(ref.shape)}: "
                                   f"sizes must match except in dimension {d}")
            if p.device != ref.device:
                raise RuntimeError(f"part {r} is on {p.device}, part 0 on {ref.device}")
            dtype = torch.promote_types(dtype, p.dtype)
        shape = list(ref.shape)
        shape[dim] = self.seq_len
        full = ref.new_empty(shape, dtype=dtype)
        for c in self._chunks:
            full.narrow(dim, c.start, c.length).copy_(parts[c.rank].narrow(dim, c.local, c.length))
        return full

    def __repr__(self) -> str:
        return f"SequenceLayout(seq_len={self.seq_len}, kind={self.kind}, sizes={self.sizes})"


__all__ = [
    "HeadShard",
    "SequenceLayout",
    "default_kv_map",
    "offsets_of",
    "partition_heads",
    "split_sizes",
]
