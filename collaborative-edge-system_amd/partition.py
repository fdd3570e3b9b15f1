"""Who owns which tokens and heads: input construction of the sequence-parallel shares.

Host-side integer arithmetic, same results as collab_infer/parallel/partition.py:
weighted largest-remainder splits (:20-68), GQA-aware head shards with shard-local
``kv_map`` (:83-160) and contiguous / zigzag sequence layouts (:166-244).  Every rank of a
real deployment evaluates these functions identically, so ownership needs no messages; on
one GPU they decide which blocks a simulated rank streams.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import torch

WeightsLike = Union[int, Sequence[float]]


def split_sizes(total: int, weights: WeightsLike, granularity: int = 1, min_units: int = 1) -> List[int]:
    """Split ``total`` into parts proportional to ``weights`` (partition.py:20-68).

    Every part is a multiple of ``granularity`` with at least ``min_units`` granules; the
    granules left after the floor of the proportional share go to the parts with the largest
    fractional remainders, lower index first on ties.
    """
    if isinstance(weights, int):
        if weights < 1:
            raise ValueError("number of parts must be >= 1")
        w = [1.0] * weights
    else:
        w = [float(x) for x in weights]
    if not w:
        raise ValueError("weights must not be empty")
    if any(not math.isfinite(x) or x <= 0 for x in w):
        raise ValueError(f"weights must be positive and finite, got {w}")
    if granularity < 1:
        raise ValueError("granularity must be >= 1")
    if total < 0 or total % granularity:
        raise ValueError(f"total={total} is not a non-negative multiple of granularity={granularity}")
    n = len(w)
    units = total // granularity
    if units < n * min_units:
        raise ValueError(
            f"cannot split {total} (granularity {granularity}) into {n} parts "
            f"with at least {min_units} unit(s) each"
        )
    spare = units - n * min_units
    weight_sum = sum(w)
    share = [spare * x / weight_sum for x in w]
    # a tiny bias keeps exact integer shares from flooring one below after rounding error
    floor = [int(math.floor(s + 1e-9)) for s in share]
    rest = spare - sum(floor)
    if rest < 0:
        floor = [int(math.floor(s)) for s in share]
        rest = spare - sum(floor)
    by_remainder = sorted(range(n), key=lambda i: (floor[i] - share[i], i))
    for i in by_remainder[:rest]:
        floor[i] += 1
    return [(f + min_units) * granularity for f in floor]


def offsets_of(sizes: Sequence[int]) -> List[int]:
    """Start offset of every part (exclusive prefix sum)."""
    starts, run = [], 0
    for s in sizes:
        starts.append(run)
        run += int(s)
    return starts


@dataclass(frozen=True)
class HeadShard:
    """Query heads owned by one rank and the KV heads they need (partition.py:83-105).

    ``kv_map[i]`` is the shard-local KV head of the ``i``-th local query head.
    """

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
    """Query head ``h`` uses KV head ``h // (num_q_heads / num_kv_heads)`` (partition.py:108-114)."""
    if num_kv_heads < 1 or num_q_heads % num_kv_heads:
        raise ValueError(f"num_q_heads={num_q_heads} must be a multiple of num_kv_heads={num_kv_heads}")
    g = num_q_heads // num_kv_heads
    return [h // g for h in range(num_q_heads)]


def partition_heads(
    num_q_heads: int,
    num_kv_heads: int,
    weights: WeightsLike,
    kv_map: Optional[Sequence[int]] = None,
) -> List[HeadShard]:
    """Partition query heads and the KV heads they need over ranks (partition.py:117-160).

    With a uniform grouping and at least as many KV heads as ranks whole KV groups are
    assigned (no KV head is duplicated); otherwise query heads are split directly and the
    KV heads they need are replicated.
    """
    mapping = default_kv_map(num_q_heads, num_kv_heads) if kv_map is None else [int(x) for x in kv_map]
    if len(mapping) != num_q_heads:
        raise ValueError("kv_map must have one entry per query head")
    if any(b < a for a, b in zip(mapping, mapping[1:])):
        raise ValueError("kv_map must be non-decreasing")
    if mapping and (mapping[0] < 0 or mapping[-1] >= num_kv_heads):
        raise ValueError("kv_map entries out of range")
    n = weights if isinstance(weights, int) else len(weights)
    uniform = (
        num_kv_heads > 0
        and num_q_heads % num_kv_heads == 0
        and mapping == default_kv_map(num_q_heads, num_kv_heads)
    )
    if uniform and num_kv_heads >= n:
        g = num_q_heads // num_kv_heads
        q_sizes = [s * g for s in split_sizes(num_kv_heads, weights)]
    else:
        if num_q_heads < n:
            raise ValueError(f"cannot split {num_q_heads} query heads over {n} ranks")
        q_sizes = split_sizes(num_q_heads, weights)
    shards = []
    for q0, qn in zip(offsets_of(q_sizes), q_sizes):
        lo, hi = mapping[q0], mapping[q0 + qn - 1] + 1
        shards.append(HeadShard(q0, qn, lo, hi - lo, tuple(m - lo for m in mapping[q0 : q0 + qn])))
    return shards


class SequenceLayout:
    """Token ownership of sequence-parallel ranks (partition.py:166-244).

    ``contiguous``: rank ``r`` owns one run of tokens.  ``zigzag``: the sequence is cut into
    ``2n`` chunks in the order ``first_0 .. first_{n-1}, second_{n-1} .. second_0`` and rank
    ``r`` owns ``first_r`` and ``second_r``, which balances causal work.
    """

    def __init__(self, seq_len: int, num_ranks: int, weights: Optional[Sequence[float]] = None,
                 kind: str = "contiguous") -> None:
        if kind not in ("contiguous", "zigzag"):
            raise ValueError(f"unknown sequence layout {kind!r}")
        self.seq_len = int(seq_len)
        self.num_ranks = int(num_ranks)
        self.kind = kind
        self.sizes = split_sizes(self.seq_len, list(weights) if weights else self.num_ranks)
        if kind == "contiguous":
            segs = [[(s, n)] for s, n in zip(offsets_of(self.sizes), self.sizes)]
        else:
            firsts = [s // 2 for s in self.sizes]
            seconds = [s - f for s, f in zip(self.sizes, firsts)]
            order = firsts + seconds[::-1]
            starts = offsets_of(order)
            n = self.num_ranks
            segs = [[(starts[r], firsts[r]), (starts[2 * n - 1 - r], seconds[r])] for r in range(n)]
        self.segments = [[(s, n) for s, n in rank_segs if n > 0] for rank_segs in segs]

    def local_len(self, rank: int) -> int:
        return self.sizes[rank]

    def indices(self, rank: int) -> torch.Tensor:
        """Global indices of the tokens of ``rank`` in local order."""
        parts = [torch.arange(s, s + n) for s, n in self.segments[rank]]
        return torch.cat(parts) if parts else torch.zeros(0, dtype=torch.long)

    def owner_of(self, index: int) -> Tuple[int, int]:
        """``(rank, local_index)`` of global token ``index``."""
        if index < 0:
            index += self.seq_len
        if not 0 <= index < self.seq_len:
            raise IndexError(f"token index {index} out of range for length {self.seq_len}")
        for rank, segs in enumerate(self.segments):
            local = 0
            for s, n in segs:
                if s <= index < s + n:
                    return rank, local + index - s
                local += n
        raise AssertionError("layout does not cover the sequence")

    def shard(self, x: torch.Tensor, rank: int, dim: int = 1) -> torch.Tensor:
        pieces = [x.narrow(dim, s, n) for s, n in self.segments[rank]]
        return pieces[0] if len(pieces) == 1 else torch.cat(pieces, dim=dim)

    def unshard(self, parts: Sequence[torch.Tensor], dim: int = 1) -> torch.Tensor:
        placed = []
        for rank, part in enumerate(parts):
            off = 0
            for s, n in self.segments[rank]:
                placed.append((s, part.narrow(dim, off, n)))
                off += n
        placed.sort(key=lambda item: item[0])
        return torch.cat([p for _, p in placed], dim=dim)

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
