"""Head-major KV cache of one attention layer, drop-in for collab_infer/models/cache.py:11-85,
with the rotary of K fused into the append.

The reference stores keys/values head-major ``[B, H, capacity, D]`` and appends token-major
``[B, n, H, D]`` blocks with two transposing copies (cache.py:51-62), right after rotating K
(``apply_rotary``, llama.py:161, 196, 205, 208).  :meth:`LayerKVCache.append_rotary` does
rotation, both copies and the position update in one kernel (``cea_kv_append``), with the
rounding points of ``apply_rotary``; :meth:`LayerKVCache.append` is the plain append.
Keys and values share one allocation when they share a shape; capacity grows by the
reference's rule (cache.py:39-49).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native as nat
from .layers import apply_rotary


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

    Keys and values are stored head-major (``k`` ``[B, Hk, capacity, Dk]``, ``v``
    ``[B, Hv, capacity, Dv]``), positions in ``[B, capacity]`` with ``-1`` in unused slots.
    When K and V share a shape - every model of the reference - they are the two halves of
    one allocation ``[2, B, H, capacity, D]`` and appends write both, rotation of K included,
    through the fused kernel (``cea_kv_append``).  A V with its own head count or head size
    (cache.py:42-43 sizes it from V) gets an allocation of its own; K is then rotated by the
    rotary kernel and both are copied in.  :meth:`view` hands out token-major
    ``[B, T, H, D]`` views of the filled prefix, which the attention kernels read in place.

    Capacity follows the reference's policy, since it decides when memory is reallocated:
    when an append does not fit, the cache grows to ``max(needed + reserve,
    int(1.5 * capacity))`` slots (cache.py:39-49) and the filled prefix moves over.
    """

    def __init__(self, reserve: int = 0) -> None:
        self.reserve = max(0, int(reserve))
        self.length = 0
        self._kv: Optional[torch.Tensor] = None    # [2, B, H, capacity, D] when K, V share a shape
        self._k: Optional[torch.Tensor] = None     # [B, Hk, capacity, Dk]
        self._v: Optional[torch.Tensor] = None     # [B, Hv, capacity, Dv]
        self._pos: Optional[torch.Tensor] = None   # [B, capacity], -1 = unused

    # -- storage -------------------------------------------------------------------------
    @property
    def k(self) -> Optional[torch.Tensor]:
        return self._k

    @property
    def v(self) -> Optional[torch.Tensor]:
        return self._v

    @property
    def pos(self) -> Optional[torch.Tensor]:
        return self._pos

    @property
    def capacity(self) -> int:
        return 0 if self._k is None else int(self._k.shape[2])

    def __len__(self) -> int:
        return self.length

    def _reserve_for(self, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor, extra: int) -> None:
        """Makes room for ``extra`` more tokens shaped like ``k`` / ``v``."""
        if k.dim() != 4 or v.dim() != 4 or tuple(v.shape[:2]) != tuple(k.shape[:2]):
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must be [B, n, H, D] "
                             "with one batch and token count")
        want = self.length + extra
        if self._k is not None and want <= self.capacity:
            return
        slots = max(want + self.reserve, int(self.capacity * 1.5))
        B, _, Hk, Dk = k.shape
        Hv, Dv = v.shape[2], v.shape[3]
        if (Hv, Dv) == (Hk, Dk):
            kv = k.new_empty((2, B, Hk, slots, Dk))
            k_new, v_new = kv[0], kv[1]
        else:
            kv, k_new, v_new = None, k.new_empty((B, Hk, slots, Dk)), v.new_empty((B, Hv, slots, Dv))
        pos_new = torch.full((B, slots), -1, dtype=torch.int64, device=k.device)
        if self.length:
            k_new[:, :, : self.length].copy_(self._k[:, :, : self.length])
            v_new[:, :, : self.length].copy_(self._v[:, :, : self.length])
            pos_new[:, : self.length].copy_(self._pos[:, : self.length])
        self._kv, self._k, self._v, self._pos = kv, k_new, v_new, pos_new

    def _write(self, k, v, pos, cos, sin) -> None:
        n = k.shape[1]
        if n == 0:
            return
        self._reserve_for(k, v, pos, n)
        if self._kv is not None and tuple(v.shape) == tuple(k.shape):
            kv_append(self._k, self._v, self._pos, self.length, k, v, pos, cos, sin)
        else:
            # V of its own shape: K through the rotary kernel, then the reference's copies
            if self._kv is not None or tuple(v.shape[2:]) != tuple(self._v.shape[1::2]):
                raise ValueError(f"v {tuple(v.shape)} does not match the cached values "
                                 f"{tuple(self._v.shape)}")
            if cos is not None:
                k = apply_rotary(k, cos, sin)
            end = self.length + n
            self._k[:, :, self.length:end].copy_(k.transpose(1, 2))
            self._v[:, :, self.length:end].copy_(v.transpose(1, 2))
            self._pos[:, self.length:end].copy_(pos)
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
        if self._k is None:
            if like_k is None or like_pos is None:
                raise RuntimeError("nothing cached yet: pass like_k and like_pos to shape empty views")
            none_k = like_k.new_empty((like_k.shape[0], 0, *like_k.shape[2:]))
            return none_k, none_k, like_pos.new_empty((like_pos.shape[0], 0))
        n = self.length
        return (self._k[:, :, :n].transpose(1, 2), self._v[:, :, :n].transpose(1, 2),
                self._pos[:, :n])

    def nbytes(self) -> int:
        """Bytes of the cached tokens' keys and values (not the unused slots)."""
        if self._k is None:
            return 0
        per_token = self._k[:, :, :1].numel() + self._v[:, :, :1].numel()
        return per_token * self._k.element_size() * self.length
