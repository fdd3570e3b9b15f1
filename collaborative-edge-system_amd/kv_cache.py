"""Head-major KV cache of one attention layer, drop-in for collab_infer/models/cache.py:11-85,
with the rotary of K fused into the append.

The reference stores keys/values head-major ``[B, H, capacity, D]`` and appends token-major
``[B, n, H, D]`` blocks with two transposing copies (cache.py:51-62), right after rotating K
(``apply_rotary``, llama.py:161, 196, 205, 208).  :meth:`LayerKVCache.append_rotary` does
rotation, both copies and the position update in one kernel (``cea_kv_append``), with the
rounding points of ``apply_rotary``; :meth:`LayerKVCache.append` is the plain append.
Keys and values share one allocation; capacity grows by the reference's rule
(cache.py:39-49).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native as nat


def kv_append(cache_k: torch.Tensor, cache_v: torch.Tensor, cache_pos: torch.Tensor, offset: int,
              k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
              cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None) -> None:
    """Writes ``k`` (rotated with ``cos``/``sin`` when given) and ``v`` ``[B, n, H, D]`` into
    the head-major caches ``[B, H, cap, D]`` at slots ``offset .. offset+n-1`` and ``pos``
    ``[B, n]`` into ``cache_pos`` ``[B, cap]``, in place."""
    if (cos is None) != (sin is None):
        raise ValueError("give both rotary tables or neither")
    if v.dtype != k.dtype or cache_k.dtype != k.dtype or cache_v.dtype != k.dtype:
        raise ValueError("k, v and the caches must share one dtype")
    nat.ops().kv_append(cache_k, cache_v, cache_pos, int(offset), k, v, pos, cos, sin)


class LayerKVCache:
    """Growable key/value cache of one attention layer on one rank (cache.py:11-85).

    Keys and values live in one device allocation ``[2, B, H, capacity, D]`` (``k`` and ``v``
    are its two head-major halves ``[B, H, capacity, D]``), positions in ``[B, capacity]``
    with ``-1`` in unused slots.  Appends write through the fused kernel (``cea_kv_append``);
    :meth:`view` hands out token-major ``[B, T, H, D]`` views of the filled prefix, which the
    attention kernels read in place.

    Capacity follows the reference's policy, since it decides when memory is reallocated:
    when an append does not fit, the cache grows to ``max(needed + reserve,
    int(1.5 * capacity))`` slots (cache.py:39-49) and the filled prefix moves over.  K and V
    must share their shape (every model of the reference has them so).
    """

    def __init__(self, reserve: int = 0) -> None:
        self.reserve = max(0, int(reserve))
        self.length = 0
        self._kv: Optional[torch.Tensor] = None    # [2, B, H, capacity, D]
        self._pos: Optional[torch.Tensor] = None   # [B, capacity], -1 = unused

    # -- storage -------------------------------------------------------------------------
    @property
    def k(self) -> Optional[torch.Tensor]:
        return None if self._kv is None else self._kv[0]

    @property
    def v(self) -> Optional[torch.Tensor]:
        return None if self._kv is None else self._kv[1]

    @property
    def pos(self) -> Optional[torch.Tensor]:
        return self._pos

    @property
    def capacity(self) -> int:
        return 0 if self._kv is None else int(self._kv.shape[3])

    def __len__(self) -> int:
        return self.length

    def _reserve_for(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor, extra: int) -> None:
        """Makes room for ``extra`` more tokens shaped like ``k`` / ``v``."""
        if tuple(v.shape) != tuple(k.shape):
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must have one shape")
        want = self.length + extra
        if self._kv is not None and want <= self.capacity:
            return
        slots = max(want + self.reserve, int(self.capacity * 1.5))
        B, _, H, D = k.shape
        kv = k.new_empty((2, B, H, slots, D))
        pos_new = torch.full((B, slots), -1, dtype=torch.int64, device=k.device)
        if self.length:
            kv[:, :, :, : self.length].copy_(self._kv[:, :, :, : self.length])
            pos_new[:, : self.length].copy_(self._pos[:, : self.length])
        self._kv, self._pos = kv, pos_new

    def _write(self, k, v, pos, cos, sin) -> None:
        n = k.shape[1]
        if n == 0:
            return
        self._reserve_for(k, v, pos, n)
        kv_append(self._kv[0], self._kv[1], self._pos, self.length, k, v, pos, cos, sin)
        self.length += n

    # -- the reference's interface ---------------------------------------------------------
    def append(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor) -> None:
        """Append token-major ``k``/``v`` (``[B, n, H, D]``) and their positions (cache.py:51-62)."""
        self._write(k, v, pos, None, None)

    def append_rotary(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor) -> None:
        """``append(apply_rotary(k, cos, sin), v, pos)`` in one kernel (``cos``/``sin``
        ``[B, n, D]`` as RotaryEmbedding returns them)."""
        self._write(k, v, pos, cos, sin)

    def view(self, like_k: Optional[torch.Tensor] = None, like_pos: Optional[torch.Tensor] = None
             ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The cached ``(k, v, pos)`` as token-major views of the filled prefix (cache.py:64-75);
        before the first append, empty tensors shaped after ``like_k`` / ``like_pos``."""
        if self._kv is None:
            if like_k is None or like_pos is None:
                raise RuntimeError("nothing cached yet: pass like_k and like_pos to shape empty views")
            none_k = like_k.new_empty((like_k.shape[0], 0, *like_k.shape[2:]))
            return none_k, none_k, like_pos.new_empty((like_pos.shape[0], 0))
        filled = self._kv[:, :, :, : self.length].transpose(2, 3)   # [2, B, T, H, D]
        return filled[0], filled[1], self._pos[:, : self.length]

    def nbytes(self) -> int:
        """Bytes of the cached tokens' keys and values (not the unused slots)."""
        if self._kv is None:
            return 0
        _, B, H, _, D = self._kv.shape
        return 2 * B * H * D * self.length * self._kv.element_size()
