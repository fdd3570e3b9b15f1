"""Head-major KV cache of one attention layer, drop-in for collab_infer/models/cache.py:11-85,
with the rotary of K fused into the append.

The reference stores keys/values head-major ``[B, H, capacity, D]`` and appends token-major
``[B, n, H, D]`` blocks with two transposing copies (cache.py:51-62), right after rotating K
(``apply_rotary``, llama.py:161, 196, 205, 208).  :meth:`LayerKVCache.append_rotary` does
rotation, both copies and the position update in one kernel (``cea_kv_append``), with the
rounding points of ``apply_rotary``; :meth:`LayerKVCache.append` is the plain append.
Growth keeps the reference's policy and copies (cache.py:39-49).
"""

from __future__ import annotations

from ctypes import byref
from typing import Optional, Tuple

import torch

from . import _native as nat


def kv_append(cache_k: torch.Tensor, cache_v: torch.Tensor, cache_pos: torch.Tensor, offset: int,
              k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
              cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None) -> None:
    """Writes ``k`` (rotated with ``cos``/``sin`` when given) and ``v`` ``[B, n, H, D]`` into
    the head-major caches ``[B, H, cap, D]`` at slots ``offset .. offset+n-1`` and ``pos``
    ``[B, n]`` into ``cache_pos`` ``[B, cap]``, in place."""
    nat.require_device(cache_k, cache_v, cache_pos, k, v, pos)
    if (cos is None) != (sin is None):
        raise ValueError("give both rotary tables or neither")
    if k.stride(-1) != 1:
        k = k.contiguous()
    if v.stride(-1) != 1:
        v = v.contiguous()
    if v.dtype != k.dtype or cache_k.dtype != k.dtype or cache_v.dtype != k.dtype:
        raise ValueError("k, v and the caches must share one dtype")
    pos = pos.to(torch.int64)
    if cos is not None:
        nat.require_device(cos, sin)
        cos, sin = cos.to(k.dtype), sin.to(k.dtype)
        cos = cos if cos.stride(-1) == 1 else cos.contiguous()
        sin = sin if sin.stride(-1) == 1 else sin.contiguous()
    a = [nat.tensor_arg(t) for t in (k, v, pos)]
    tabs = [nat.tensor_arg(cos), nat.tensor_arg(sin)] if cos is not None else None
    dst = [nat.tensor_arg(t) for t in (cache_k, cache_v, cache_pos)]
    rc = nat.load_library().cea_kv_append(
        byref(a[0]), byref(a[1]), byref(a[2]),
        byref(tabs[0]) if tabs else None, byref(tabs[1]) if tabs else None,
        byref(dst[0]), byref(dst[1]), byref(dst[2]), int(offset), nat.stream_of(k.device))
    nat.check(rc, "kv_append")


class LayerKVCache:
    """Growable key/value cache of one attention layer on one rank (cache.py:11-85).

    Keys/values are stored head-major ``[B, H_local, capacity, D]``; :meth:`view` returns
    token-major ``[B, T, H_local, D]`` views of the same memory.  Positions of the cached
    tokens are kept as ``[B, capacity]`` (``-1`` in unused slots).
    """

    def __init__(self, reserve: int = 0) -> None:
        self.k: Optional[torch.Tensor] = None  # [B, H, capacity, D]
        self.v: Optional[torch.Tensor] = None
        self.pos: Optional[torch.Tensor] = None  # [B, capacity]
        self.length = 0
        self.reserve = max(0, int(reserve))

    def __len__(self) -> int:
        return self.length

    @property
    def capacity(self) -> int:
        return 0 if self.k is None else self.k.shape[2]

    def _grow(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor, needed: int) -> None:
        # cache.py:39-49: max(needed + reserve, 1.5 x capacity) slots, old content copied,
        # unused position slots -1
        capacity = max(needed + self.reserve, int(self.capacity * 1.5))
        B, _, H, D = k.shape
        new_k = k.new_empty((B, H, capacity, D))
        new_v = v.new_empty((B, v.shape[2], capacity, v.shape[3]))
        new_pos = pos.new_full((B, capacity), -1, dtype=torch.int64)
        if self.length:
            new_k[:, :, : self.length] = self.k[:, :, : self.length]
            new_v[:, :, : self.length] = self.v[:, :, : self.length]
            new_pos[:, : self.length] = self.pos[:, : self.length]
        self.k, self.v, self.pos = new_k, new_v, new_pos

    def _append(self, k, v, pos, cos, sin) -> None:
        n = k.shape[1]
        if n == 0:
            return
        if self.k is None or self.length + n > self.capacity:
            self._grow(k, v, pos, self.length + n)
        kv_append(self.k, self.v, self.pos, self.length, k, v, pos, cos, sin)
        self.length += n

    def append(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor) -> None:
        """Append token-major ``k``/``v`` (``[B, n, H, D]``) and their positions (cache.py:51-62)."""
        self._append(k, v, pos, None, None)

    def append_rotary(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor) -> None:
        """``append(apply_rotary(k, cos, sin), v, pos)`` in one kernel (``cos``/``sin``
        ``[B, n, D]`` as RotaryEmbedding returns them)."""
        self._append(k, v, pos, cos, sin)

    def view(self, like_k: Optional[torch.Tensor] = None, like_pos: Optional[torch.Tensor] = None
             ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Cached ``(k, v, pos)`` as token-major views (cache.py:64-75)."""
        if self.k is None:
            if like_k is None or like_pos is None:
                raise RuntimeError("empty cache: provide templates to build empty views")
            empty = like_k.new_empty((like_k.shape[0], 0) + tuple(like_k.shape[2:]))
            return empty, empty, like_pos.new_empty((like_pos.shape[0], 0))
        n = self.length
        return self.k[:, :, :n].transpose(1, 2), self.v[:, :, :n].transpose(1, 2), self.pos[:, :n]

    def nbytes(self) -> int:
        if self.k is None:
            return 0
        per_token = (self.k[:, :, :1].numel() + self.v[:, :, :1].numel()) * self.k.element_size()
        return per_token * self.length
