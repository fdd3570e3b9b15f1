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


def pack_partial(out, lse):
    """sequence_parallel.py:275: the all-gather message ``[B, Sq, H, D+1]`` (out | lse)."""
    return torch.cat([out, lse.transpose(1, 2).unsqueeze(-1)], dim=-1)


def merge_packed(parts, out_dtype):
    """sequence_parallel.py:277-280: unpack every gathered message, merge in rank order,
    cast to the query dtype."""
    D = parts[0].shape[-1] - 1
    outs = [p[..., :D] for p in parts]
    lses = [p[..., D].transpose(1, 2) for p in parts]
    out, _ = merge_many(outs, lses) if len(parts) > 1 else (outs[0], lses[0])
    return out.to(out_dtype)


def ulysses_scatter(shards, head_shards, rank: int):
    """sequence_parallel.py:163-178 for rank ``rank``.  ``shards[j] = (q_j, k_j, v_j, pos_j)``
    is rank j's sequence shard; the all_to_all delivers to ``rank`` what every rank j puts in
    its send list at index ``rank``.  Returns ``(q_f, k_f, v_f, pos_f)``."""
    received = []
    for q, k, v, _ in shards:  # what rank j sends
        sends = [torch.cat([q[:, :, sh.q_start : sh.q_start + sh.q_count],
                            k[:, :, sh.kv_start : sh.kv_start + sh.kv_count],
                            v[:, :, sh.kv_start : sh.kv_start + sh.kv_count]], dim=2).contiguous()
                 for sh in head_shards]
        received.append(sends[rank])
    full = torch.cat(received, dim=1) if len(shards) > 1 else received[0]
    me = head_shards[rank]
    q_f, k_f, v_f = full.split([me.q_count, me.kv_count, me.kv_count], dim=2)
    pos_f = torch.cat([s[3] for s in shards], dim=1)
    return q_f, k_f, v_f, pos_f


def ulysses_gather(out_heads, seq_sizes: Sequence[int], rank: int):
    """sequence_parallel.py:182-194 for rank ``rank``: ``out_heads[j]`` is rank j's head output
    over the whole sequence; rank j sends token slice i to rank i."""
    starts = [sum(seq_sizes[:i]) for i in range(len(seq_sizes))]
    back = [o[:, starts[rank] : starts[rank] + seq_sizes[rank]].contiguous() for o in out_heads]
    return torch.cat(back, dim=2) if len(back) > 1 else back[0]


def ulysses_local(q_f, k_f, v_f, pos_f, kv_map=None, *, causal=True, scale=None):
    """sequence_parallel.py:237: the head-sharded local attention after the scatter."""
    return plain_attention(q_f, k_f, v_f, pos_f, pos_f, causal=causal, scale=scale, kv_map=kv_map)


def wire_round(t: torch.Tensor, activation_dtype) -> torch.Tensor:
    """A tensor after a compressed transfer (distributed/comm.py:275-290, 468-486): floating
    tensors travel in ``activation_dtype`` only when it is narrower than their own dtype,
    float16 saturating at +-65504 (to_wire), and are cast back on arrival."""
    if activation_dtype is None or not t.dtype.is_floating_point:
        return t
    if torch.empty(0, dtype=activation_dtype).element_size() >= t.element_size():
        return t
    w = t.clamp(-65504.0, 65504.0) if activation_dtype == torch.float16 else t
    return w.to(activation_dtype).to(t.dtype)
