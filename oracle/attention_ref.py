"""CPU restatement of collab_infer/parallel/attention.py (test infrastructure only).

The CPU route of the reference (``_flash_lse``, attention.py:163-181) is restated with the
same ATen operator, the same mask-mode decision (``_mask_mode`` :116-127), the same query
chunking (``_plan`` :130-141, ``MASK_CHUNK_ELEMENTS`` :39) and the same empty-row fix-up
(:173-176).  ``math_lse`` restates the materialised-scores route (:184-198), used for
f64-exact checks and by ``attention_with_lse(..., route="math")``.
"""

from __future__ import annotations

import math
from typing import Iterator, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

MASK_CHUNK_ELEMENTS = 1 << 22  # attention.py:39
_FLASH_CPU = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu  # attention.py:41


def acc_dtype(dtype: torch.dtype) -> torch.dtype:
    """attention.py:56-57."""
    return torch.float64 if dtype == torch.float64 else torch.float32


def _map_list(kv_map) -> Optional[List[int]]:
    if kv_map is None:
        return None
    if isinstance(kv_map, torch.Tensor):
        return [int(x) for x in kv_map.tolist()]
    return [int(x) for x in kv_map]


def expand_heads(x: torch.Tensor, hq: int, kv_map=None) -> torch.Tensor:
    """attention.py:68-82: KV head h of the result serves query head h."""
    m = _map_list(kv_map)
    hkv = x.shape[2]
    if m is None:
        if hkv == hq:
            return x
        if hq % hkv:
            raise ValueError(f"{hq} query heads cannot share {hkv} KV heads evenly")
        return x.repeat_interleave(hq // hkv, dim=2)
    if len(m) != hq:
        raise ValueError("kv_map must have one entry per query head")
    if hkv == hq and m == list(range(hq)):
        return x
    return x.index_select(2, torch.tensor(m, dtype=torch.long))


def group_of(hq: int, hkv: int, kv_map=None) -> Optional[int]:
    """attention.py:85-93."""
    if hkv < 1 or hq % hkv:
        return None
    g = hq // hkv
    m = _map_list(kv_map)
    return g if m is None or m == [h // g for h in range(hq)] else None


def visible(q_pos: torch.Tensor, k_pos: torch.Tensor, causal: bool = True) -> torch.Tensor:
    """attention.py:96-101: ``[B, 1, Sq, Sk]`` bool."""
    ok = (k_pos >= 0)[:, None, None, :]
    if causal:
        ok = ok & (k_pos[:, None, None, :] <= q_pos[:, None, :, None])
    return ok.expand(q_pos.shape[0], 1, q_pos.shape[1], k_pos.shape[1])


def nothing_visible(q_pos: torch.Tensor, k_pos: torch.Tensor, causal: bool = True) -> bool:
    """attention.py:104-113 (fully_masked)."""
    if k_pos.numel() == 0 or q_pos.numel() == 0:
        return True
    good = k_pos[k_pos >= 0]
    if good.numel() == 0:
        return True
    return bool(causal and q_pos.max() < good.min())


def dispatch_mode(q_pos: torch.Tensor, k_pos: torch.Tensor, causal: bool) -> str:
    """attention.py:116-127: "none", "causal" (aligned prefill) or "mask"."""
    if not bool((k_pos >= 0).all()):
        return "mask"
    if not causal:
        return "none"
    if bool((q_pos >= 0).all()) and bool((k_pos.amax(dim=1) <= q_pos.amin(dim=1)).all()):
        return "none"
    if q_pos.shape == k_pos.shape and torch.equal(q_pos, k_pos):
        if q_pos.shape[1] == 1 or bool((q_pos[:, 1:] - q_pos[:, :-1] == 1).all()):
            return "causal"
    return "mask"


def query_chunks(q_pos, k_pos, causal) -> Iterator[Tuple[int, int, str, Optional[torch.Tensor]]]:
    """attention.py:130-141."""
    B, Sq = q_pos.shape
    Sk = k_pos.shape[1]
    mode = dispatch_mode(q_pos, k_pos, causal)
    if mode != "mask":
        yield 0, Sq, mode, None
        return
    rows = max(1, MASK_CHUNK_ELEMENTS // max(1, B * Sk))
    for lo in range(0, Sq, rows):
        hi = min(Sq, lo + rows)
        yield lo, hi, mode, visible(q_pos[:, lo:hi], k_pos, causal)


def _kv_for(k, v, hq, kv_map, native_gqa: bool):
    """attention.py:144-149."""
    g = group_of(hq, k.shape[2], kv_map)
    if g is None or (g > 1 and not native_gqa):
        return expand_heads(k, hq, kv_map), expand_heads(v, hq, kv_map), 1
    return k, v, g


def empty_result(q: torch.Tensor, acc: torch.dtype):
    """attention.py:152-157."""
    B, Sq, Hq, D = q.shape
    return torch.zeros(B, Sq, Hq, D, dtype=acc), torch.full((B, Hq, Sq), float("-inf"), dtype=acc)


def empty_rows_fixup(o, l, mask):
    """attention.py:173-176: the CPU flash op reports lse 0 for a row with no visible key;
    such rows become out 0, lse -inf."""
    empty = ~mask.any(dim=-1)
    return o.masked_fill(empty.unsqueeze(-1), 0.0), l.masked_fill(empty, float("-inf"))


def flash_lse(q, k, v, q_pos, k_pos, causal, scale, kv_map, acc):
    """attention.py:163-181: the CPU flash kernel over query chunks with an additive bias."""
    k, v, _ = _kv_for(k, v, q.shape[2], kv_map, native_gqa=True)
    qh, kh, vh = (t.to(acc).transpose(1, 2) for t in (q, k, v))
    outs, lses = [], []
    for lo, hi, mode, mask in query_chunks(q_pos, k_pos, causal):
        bias = None
        if mask is not None:
            bias = torch.zeros(mask.shape, dtype=acc).masked_fill(~mask, float("-inf"))
        o, l = _FLASH_CPU(qh[:, :, lo:hi], kh, vh, 0.0, mode == "causal", attn_mask=bias, scale=scale)
        if mask is not None:
            o, l = empty_rows_fixup(o, l, mask)
        outs.append(o)
        lses.append(l)
    out = outs[0] if len(outs) == 1 else torch.cat(outs, dim=2)
    lse = lses[0] if len(lses) == 1 else torch.cat(lses, dim=2)
    return out.transpose(1, 2), lse


def math_lse(q, k, v, q_pos, k_pos, causal, scale, kv_map, acc):
    """attention.py:184-198: materialised scores, grouped heads without copying K/V."""
    B, Sq, Hq, D = q.shape
    k, v, g = _kv_for(k, v, Hq, kv_map, native_gqa=True)
    Hkv = k.shape[2]
    qg = q.to(acc).permute(0, 2, 1, 3).reshape(B, Hkv, g * Sq, D)
    kh, vh = k.to(acc).transpose(1, 2), v.to(acc).transpose(1, 2)
    s = torch.matmul(qg, kh.transpose(-1, -2)) * scale
    m = visible(q_pos, k_pos, causal).repeat(1, 1, g, 1)
    s = s.masked_fill(~m, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
    out = torch.matmul(torch.exp(s - safe.unsqueeze(-1)), vh)
    return out.reshape(B, Hq, Sq, D).transpose(1, 2), lse.reshape(B, Hq, Sq)


def attention_with_lse(q, k, v, q_pos, k_pos, *, causal=True, scale=None, kv_map=None,
                       kv_block=None, route: str = "flash"):
    """attention.py:201-239 on CPU tensors.  ``route="flash"`` is the reference's CPU route,
    ``route="math"`` its portable route."""
    acc = acc_dtype(q.dtype)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    Sk = k.shape[1]
    if Sk == 0 or q.shape[1] == 0:
        return empty_result(q, acc)
    if kv_block is not None and kv_block < Sk:
        out = lse = None
        for lo in range(0, Sk, kv_block):
            hi = min(lo + kv_block, Sk)
            kp = k_pos[:, lo:hi]
            if nothing_visible(q_pos, kp, causal):
                continue
            o, l = attention_with_lse(q, k[:, lo:hi], v[:, lo:hi], q_pos, kp, causal=causal,
                                      scale=scale, kv_map=kv_map, route=route)
            out, lse = (o, l) if out is None else merge_pair(out, lse, o, l)
        return empty_result(q, acc) if out is None else (out, lse)
    fn = flash_lse if route == "flash" else math_lse
    return fn(q, k, v, q_pos, k_pos, causal, scale, kv_map, acc)


def merge_pair(out_a, lse_a, out_b, lse_b):
    """attention.py:242-250."""
    lse = torch.logaddexp(lse_a, lse_b)
    safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
    wa = torch.exp(lse_a - safe).transpose(1, 2).unsqueeze(-1)
    wb = torch.exp(lse_b - safe).transpose(1, 2).unsqueeze(-1)
    return out_a * wa + out_b * wb, lse


def merge_many(outs: Sequence[torch.Tensor], lses: Sequence[torch.Tensor]):
    """attention.py:253-264."""
    if len(outs) == 1:
        return outs[0], lses[0]
    st = torch.stack(list(lses))
    lse = torch.logsumexp(st, dim=0)
    safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
    w = torch.exp(st - safe)
    out = sum(o * wi.transpose(1, 2).unsqueeze(-1) for o, wi in zip(outs, w))
    return out, lse


def plain_attention(q, k, v, q_pos, k_pos, *, causal=True, scale=None, kv_map=None, kv_block=None):
    """attention.py:270-301: SDPA per query chunk, rows without visible keys set to 0."""
    Sk = k.shape[1]
    if kv_block is not None and kv_block < Sk:
        out, _ = attention_with_lse(q, k, v, q_pos, k_pos, causal=causal, scale=scale,
                                    kv_map=kv_map, kv_block=kv_block)
        return out.to(q.dtype)
    if Sk == 0 or q.shape[1] == 0:
        return torch.zeros_like(q)
    k, v, g = _kv_for(k, v, q.shape[2], kv_map, native_gqa=True)
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    extra = {"enable_gqa": True} if g > 1 else {}
    outs = []
    for lo, hi, mode, mask in query_chunks(q_pos, k_pos, causal):
        o = F.scaled_dot_product_attention(qh[:, :, lo:hi], kh, vh, attn_mask=mask,
                                           is_causal=mode == "causal", scale=scale, **extra)
        if mask is not None:
            o = o.masked_fill(~mask.any(dim=-1, keepdim=True), 0.0)
        outs.append(o)
    out = outs[0] if len(outs) == 1 else torch.cat(outs, dim=2)
    return out.transpose(1, 2)
