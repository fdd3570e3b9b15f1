"""CPU restatement of one rank's sequence-parallel shares (test infrastructure only).

The collectives are replaced by direct access to every rank's shard, which is exactly what
the messages deliver; the compute order (ring step order, skip rule, merge order) follows
collab_infer/parallel/sequence_parallel.py.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import torch

from .attention_ref import attention_with_lse, merge_many, merge_pair, nothing_visible, plain_attention


def ring_share(q, q_pos, blocks: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]], rank: int,
               *, causal=True, scale=None, kv_map=None, kv_block=None, with_lse=False):
    """sequence_parallel.py:94-130 for rank ``rank``: blocks by source rank, visited in the
    order ``(rank - step) mod n``; fully hidden blocks skipped; online pairwise merge."""
    n = len(blocks)
    if n == 1:
        out, lse = attention_with_lse(q, *blocks[0][:2], q_pos, blocks[0][2], causal=causal,
                                      scale=scale, kv_map=kv_map, kv_block=kv_block)
        return (out, lse) if with_lse else out.to(q.dtype)
    out = lse = None
    for step in range(n):
        k, v, pos = blocks[(rank - step) % n]
        if nothing_visible(q_pos, pos, causal):
            continue
        o, l = attention_with_lse(q, k, v, q_pos, pos, causal=causal, scale=scale, kv_map=kv_map,
                                  kv_block=kv_block)
        out, lse = (o, l) if out is None else merge_pair(out, lse, o, l)
    if out is None:
        return (torch.zeros_like(q, dtype=torch.float32), None) if with_lse else torch.zeros_like(q)
    return (out, lse) if with_lse else out.to(q.dtype)


def distributed_kv_share(q, q_pos, parts, *, causal=True, scale=None, kv_map=None, kv_block=None,
                         with_parts=False):
    """sequence_parallel.py:270-280: each rank's partial, merged in rank order."""
    partial = [attention_with_lse(q, k, v, q_pos, p, causal=causal, scale=scale, kv_map=kv_map,
                                  kv_block=kv_block) for k, v, p in parts]
    if len(partial) == 1:
        out = partial[0][0]
        lse = partial[0][1]
    else:
        out, lse = merge_many([p[0] for p in partial], [p[1] for p in partial])
    res = out.to(q.dtype)
    return (res, lse, partial) if with_parts else res


def ulysses_local(q_f, k_f, v_f, pos_f, kv_map=None, *, causal=True, scale=None):
    """sequence_parallel.py:237: the head-sharded local attention after the scatter."""
    return plain_attention(q_f, k_f, v_f, pos_f, pos_f, causal=causal, scale=scale, kv_map=kv_map)
