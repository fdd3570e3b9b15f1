"""Seeded synthetic inputs of the five workloads of the attention / layer-op path, and their
algorithmic work counts.

Inputs are drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in f32 (as the
reference's tests do, tests/test_sequence_parallel.py:18-22), then cast and moved, so the
CPU oracle and the GPU see bit-identical inputs.

* ``attn_f32_split``   - f32 attention B=1, 8/8 heads, S=512, D=64, causal, plus a 2-way KV
  split merged by LSE.
* ``layer_ops``        - bf16 RMSNorm + rotary on a 4096 x 4096 activation viewed as
  32 heads x 128 (theta 1e4, positions 0..4095) and SiLU-gate on 4096 x 14336 gate/up.
* ``ring_share``       - rank 0 of a 4-rank zigzag ring over 32768 tokens: 8192 local queries
  (positions 0..4095 and 28672..32767), 32/8 GQA heads, D=128, bf16; four 8192-token KV
  blocks streamed in ring order 0, 3, 2, 1 (sequence_parallel.py:107-110).
* ``kv_decode``        - distributed-KV decode: B=32, one query token, 32/8 heads, D=128,
  bf16; head-major cache ``[32, 8, 32768, 128]`` (models/cache.py:11-20) with valid lengths
  uniform in [1024, 32768]; four contiguous partitions with weights 0.4/0.3/0.2/0.1.
* ``ulysses_share``    - rank 0 of an 8-way Ulysses split of a 64/16-head model: 65536 tokens,
  8/2 heads, D=128, bf16, causal, 4 packed sequences followed by right padding.
* ``projections``      - the fused gate/up (4096 tokens, 4096 -> 2 x 14336, SiLU) and Q/K/V
  (8192 tokens, 4096 -> 32/8/8 heads x 128) projections of a Llama-3-8B-shaped layer, bf16.
* ``kv_append``        - one rank's 8192-token prefill chunk (8 KV heads, D=128, bf16, theta
  1e4) rotated and appended into a head-major cache that already holds 8192 tokens.
* ``prefill_chunk``    - one 128-token chunk of a chunked prefill (engine.py:91-92) at batch
  1 against the 32768 keys it sees (the cache before it and itself), 32/8 heads, D=128, bf16,
  causal: few query blocks against a long key block.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .partition import SequenceLayout, partition_heads, split_sizes


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def _randn(g: torch.Generator, *shape, dtype=torch.bfloat16, device="cpu") -> torch.Tensor:
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype).to(device)


def visible_pairs(q_pos: torch.Tensor, k_pos: torch.Tensor, causal: bool = True) -> int:
    """Exact number of visible (query, key) pairs for one head of a ``[1, S]`` position pair."""
    kp = k_pos.reshape(-1).to(torch.int64).cpu()
    kp = torch.sort(kp[kp >= 0]).values
    qp = q_pos.reshape(-1).to(torch.int64).cpu()
    if not causal:
        return int(kp.numel()) * int(qp.numel())
    return int(torch.searchsorted(kp, qp, right=True).sum())


# --------------------------------------------------------------------------------------
@dataclass
class AttnF32Split:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    pos: torch.Tensor
    scale: float
    split: int
    flop: int


def attn_f32_split(device="cpu", seed: int = 0) -> AttnF32Split:
    g = _gen(seed)
    B, H, S, D = 1, 8, 512, 64
    q = _randn(g, B, S, H, D, dtype=torch.float32, device=device)
    k = _randn(g, B, S, H, D, dtype=torch.float32, device=device)
    v = _randn(g, B, S, H, D, dtype=torch.float32, device=device)
    pos = torch.arange(S, device=device).view(1, S)
    flop = 4 * D * H * S * (S + 1) // 2
    return AttnF32Split(q, k, v, pos, 1.0 / 8.0, 256, flop)


# --------------------------------------------------------------------------------------
@dataclass
class LayerOps:
    x: torch.Tensor
    weight: torch.Tensor
    positions: torch.Tensor
    gate: torch.Tensor
    up: torch.Tensor
    heads: int = 32
    head_dim: int = 128
    theta: float = 1e4
    eps: float = 1e-5

    @property
    def rmsnorm_rope_bytes(self) -> int:
        # x read + y written + weight (tables generated in-kernel)
        return 2 * self.x.numel() * 2 + self.weight.numel() * 2

    @property
    def silu_bytes(self) -> int:
        return 3 * self.gate.numel() * 2


def layer_ops(device="cpu", seed: int = 0, tokens: int = 4096, hidden: int = 4096,
              inter: int = 14336) -> LayerOps:
    g = _gen(seed)
    x = _randn(g, tokens, hidden, device=device)
    w = (1.0 + 0.02 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(device)
    gate = _randn(g, tokens, inter, device=device)
    up = _randn(g, tokens, inter, device=device)
    pos = torch.arange(tokens, device=device).view(1, tokens)
    return LayerOps(x, w, pos, gate, up)


# --------------------------------------------------------------------------------------
@dataclass
class Projections:
    """The fused projections of a Llama-3-8B-shaped layer (hidden 4096, 32/8 heads x 128,
    intermediate 14336) on one device: the gate/up projection of 4096 tokens with SiLU, and
    the Q/K/V projection of the ring share's 8192 local tokens."""
    x_mlp: torch.Tensor      # [4096, 4096]
    w_gate_up: torch.Tensor  # [2 * 14336, 4096], gate rows first
    x_attn: torch.Tensor     # [8192, 4096]
    w_qkv: torch.Tensor      # [(32 + 8 + 8) * 128, 4096]
    inter: int = 14336

    @property
    def flop_gate_up(self) -> int:
        return 2 * self.x_mlp.shape[0] * self.x_mlp.shape[1] * self.w_gate_up.shape[0]

    @property
    def flop_qkv(self) -> int:
        return 2 * self.x_attn.shape[0] * self.x_attn.shape[1] * self.w_qkv.shape[0]


def projections(device="cpu", seed: int = 0, mlp_tokens: int = 4096, attn_tokens: int = 8192,
                hidden: int = 4096, inter: int = 14336, hq: int = 32, hkv: int = 8,
                d: int = 128) -> Projections:
    g = _gen(seed)
    scale = hidden ** -0.5
    x_mlp = _randn(g, mlp_tokens, hidden, device=device)
    w_gu = (torch.randn(2 * inter, hidden, generator=g) * scale).to(torch.bfloat16).to(device)
    x_attn = _randn(g, attn_tokens, hidden, device=device)
    w_qkv = (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) * scale).to(torch.bfloat16).to(device)
    return Projections(x_mlp, w_gu, x_attn, w_qkv, inter)


# --------------------------------------------------------------------------------------
@dataclass
class RingShare:
    q: torch.Tensor                        # [1, 8192, 32, 128]
    q_pos: torch.Tensor                    # [1, 8192]
    blocks: List[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]  # by source rank
    layout: SequenceLayout
    rank: int
    kv_sizes: List[int]
    pairs_per_step: List[int]              # in ring order

    @property
    def ring_order(self) -> List[int]:
        n = self.layout.num_ranks
        return [(self.rank - s) % n for s in range(n)]

    @property
    def flop(self) -> int:
        return 4 * self.q.shape[-1] * self.q.shape[2] * sum(self.pairs_per_step)


def ring_share(device="cpu", seed: int = 0, seq_len: int = 32768, sp: int = 4, rank: int = 0,
               hq: int = 32, hkv: int = 8, d: int = 128, dtype=torch.bfloat16) -> RingShare:
    g = _gen(seed)
    layout = SequenceLayout(seq_len, sp, kind="zigzag")
    s_loc = layout.sizes[rank]
    q = _randn(g, 1, s_loc, hq, d, dtype=dtype, device=device)
    blocks = []
    for r in range(sp):
        n = layout.sizes[r]
        k = _randn(g, 1, n, hkv, d, dtype=dtype, device=device)
        v = _randn(g, 1, n, hkv, d, dtype=dtype, device=device)
        blocks.append((k, v, layout.indices(r).view(1, n).to(device)))
    q_pos = layout.indices(rank).view(1, s_loc).to(device)
    order = [(rank - s) % sp for s in range(sp)]
    pairs = [visible_pairs(q_pos, blocks[r][2]) for r in order]
    return RingShare(q, q_pos, blocks, layout, rank, list(layout.sizes), pairs)


# --------------------------------------------------------------------------------------
@dataclass
class KVDecode:
    q: torch.Tensor                 # [B, 1, Hq, D]
    q_pos: torch.Tensor             # [B, 1]
    cache_k: torch.Tensor           # [B, Hkv, cap, D] head-major
    cache_v: torch.Tensor
    k_pos: torch.Tensor             # [B, cap] (-1 = unused slot)
    lengths: torch.Tensor           # [B]
    part_sizes: List[int]
    batch: List[int]                # which sequences of the full workload these rows are

    def partitions(self) -> List[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
        """Token-major views ``[B, s_p, Hkv, D]`` of each partition (no copies, cache.py:64-74)."""
        out, start = [], 0
        for n in self.part_sizes:
            k = self.cache_k[:, :, start : start + n].transpose(1, 2)
            v = self.cache_v[:, :, start : start + n].transpose(1, 2)
            out.append((k, v, self.k_pos[:, start : start + n]))
            start += n
        return out

    @property
    def kv_bytes(self) -> int:
        hkv, d = self.cache_k.shape[1], self.cache_k.shape[3]
        return int(self.lengths.sum()) * hkv * d * 2 * self.cache_k.element_size()

    @property
    def bytes(self) -> int:
        """Algorithmic HBM bytes of one decode + merge step: valid K/V, the query, every
        partition's f32 (out, lse) written and read back by the merge, the final output."""
        B, _, hq, d = self.q.shape
        n = len(self.part_sizes)
        q_b = self.q.numel() * self.q.element_size()
        partial = n * (B * hq * d * 4 + B * hq * 4)
        return self.kv_bytes + q_b + 2 * partial + q_b


def kv_decode(device="cpu", seed: int = 0, batch: Optional[Sequence[int]] = None, B: int = 32,
              hq: int = 32, hkv: int = 8, d: int = 128, cap: int = 32768,
              weights=(0.4, 0.3, 0.2, 0.1), min_len: int = 1024,
              dtype=torch.bfloat16) -> KVDecode:
    """Cache contents are drawn per sequence (generator ``seed + 1 + b``) for its valid slots
    only, so any subset of sequences is reproducible on its own; unused slots hold zeros."""
    g = _gen(seed)
    lengths_all = torch.randint(min_len, cap + 1, (B,), generator=g)
    q_all = torch.randn(B, 1, hq, d, generator=g, dtype=torch.float32)
    rows = list(range(B)) if batch is None else [int(b) for b in batch]
    nb = len(rows)
    cache_k = torch.zeros(nb, hkv, cap, d, dtype=dtype, device=device)
    cache_v = torch.zeros(nb, hkv, cap, d, dtype=dtype, device=device)
    for i, b in enumerate(rows):
        L = int(lengths_all[b])
        gb = _gen(seed + 1 + b)
        cache_k[i, :, :L] = torch.randn(hkv, L, d, generator=gb).to(dtype).to(device)
        cache_v[i, :, :L] = torch.randn(hkv, L, d, generator=gb).to(dtype).to(device)
    lengths = lengths_all[rows]
    slots = torch.arange(cap).view(1, cap)
    k_pos = torch.where(slots < lengths.view(-1, 1), slots, torch.full_like(slots, -1)).to(device)
    q = q_all[rows].to(dtype).to(device)
    q_pos = (lengths - 1).view(-1, 1).to(device)
    return KVDecode(q, q_pos, cache_k, cache_v, k_pos, lengths, split_sizes(cap, list(weights)),
                    rows)


# --------------------------------------------------------------------------------------
@dataclass
class UlyssesShare:
    q: torch.Tensor        # [1, S, 8, 128]
    k: torch.Tensor        # [1, S, 2, 128]
    v: torch.Tensor
    pos: torch.Tensor      # [1, S]: 0..L-1 then -1
    lengths: List[int]
    kv_map: Optional[Tuple[int, ...]]

    @property
    def valid(self) -> int:
        return sum(self.lengths)

    @property
    def flop(self) -> int:
        L = self.valid
        return 4 * self.q.shape[-1] * self.q.shape[2] * L * (L + 1) // 2


def ulysses_share(device="cpu", seed: int = 0, seq_len: int = 65536, model_heads=(64, 16),
                  sp: int = 8, rank: int = 0, d: int = 128, n_seq: int = 4,
                  dtype=torch.bfloat16) -> UlyssesShare:
    g = _gen(seed)
    lengths = [int(x) for x in torch.randint(1, seq_len // n_seq + 1, (n_seq,), generator=g)]
    shard = partition_heads(model_heads[0], model_heads[1], sp)[rank]
    q = _randn(g, 1, seq_len, shard.q_count, d, dtype=dtype, device=device)
    k = _randn(g, 1, seq_len, shard.kv_count, d, dtype=dtype, device=device)
    v = _randn(g, 1, seq_len, shard.kv_count, d, dtype=dtype, device=device)
    # positions of packed tokens: where(mask, cumsum(mask) - 1, -1) (engine/engine.py:328-329)
    mask = torch.arange(seq_len) < sum(lengths)
    pos = torch.where(mask, torch.cumsum(mask.to(torch.int64), 0) - 1, torch.full((seq_len,), -1))
    kv_map = tuple(shard.kv_map)
    return UlyssesShare(q, k, v, pos.view(1, seq_len).to(device), lengths, kv_map)


__all__ = [
    "AttnF32Split",
    "KVDecode",
    "LayerOps",
    "RingShare",
    "UlyssesShare",
    "attn_f32_split",
    "kv_decode",
    "layer_ops",
    "ring_share",
    "ulysses_share",
    "visible_pairs",
]


@dataclass
class KVAppend:
    k: torch.Tensor          # [1, n, Hkv, D] token-major, before the rotary
    v: torch.Tensor
    pos: torch.Tensor        # [1, n]
    cos: torch.Tensor        # [1, n, D]
    sin: torch.Tensor
    cache_k: torch.Tensor    # [1, Hkv, capacity, D]
    cache_v: torch.Tensor
    cache_pos: torch.Tensor  # [1, capacity]
    offset: int

    @property
    def bytes(self) -> int:
        # k, v read and written once, the tables read once (shared by the heads),
        # positions read and written
        kv = self.k.numel() * self.k.element_size()
        tab = self.cos.numel() * self.cos.element_size()
        return 4 * kv + 2 * tab + 2 * self.pos.numel() * 8


def kv_append(device="cpu", seed: int = 0, n: int = 8192, heads: int = 8, head_dim: int = 128,
              cached: int = 8192, theta: float = 1e4) -> KVAppend:
    g = _gen(seed)
    k = _randn(g, 1, n, heads, head_dim, device=device)
    v = _randn(g, 1, n, heads, head_dim, device=device)
    pos = torch.arange(cached, cached + n, device=device).view(1, n)
    half = torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim
    inv = 1.0 / (theta ** half)
    freqs = pos.to("cpu").to(torch.float32).unsqueeze(-1) * inv
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16).to(device), emb.sin().to(torch.bfloat16).to(device)
    cap = cached + n
    cache_k = torch.zeros(1, heads, cap, head_dim, dtype=torch.bfloat16, device=device)
    cache_v = torch.zeros_like(cache_k)
    cache_pos = torch.full((1, cap), -1, dtype=torch.int64, device=device)
    return KVAppend(k, v, pos, cos, sin, cache_k, cache_v, cache_pos, cached)


# --------------------------------------------------------------------------------------
@dataclass
class PrefillChunk:
    q: torch.Tensor        # [B, chunk, hq, d]
    k: torch.Tensor        # [B, keys, hkv, d]
    v: torch.Tensor
    q_pos: torch.Tensor    # [B, chunk]: the last chunk positions
    k_pos: torch.Tensor    # [B, keys]: 0..keys-1

    @property
    def flop(self) -> int:
        B, S, H, D = self.q.shape
        keys = self.k.shape[1]
        return 4 * D * H * B * sum(keys - S + 1 + i for i in range(S))


def prefill_chunk(device="cpu", seed: int = 0, B: int = 1, chunk: int = 128, keys: int = 32768,
                  hq: int = 32, hkv: int = 8, d: int = 128, dtype=torch.bfloat16) -> PrefillChunk:
    g = _gen(seed)
    q = _randn(g, B, chunk, hq, d, dtype=dtype, device=device)
    k = _randn(g, B, keys, hkv, d, dtype=dtype, device=device)
    v = _randn(g, B, keys, hkv, d, dtype=dtype, device=device)
    k_pos = torch.arange(keys).repeat(B, 1).to(device)
    q_pos = torch.arange(keys - chunk, keys).repeat(B, 1).to(device)
    return PrefillChunk(q, k, v, q_pos, k_pos)
