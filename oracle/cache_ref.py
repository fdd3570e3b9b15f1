"""CPU restatement of the reference's per-layer KV cache (test infrastructure only).

Follows collab_infer/models/cache.py:11-85: head-major ``[B, H, capacity, D]`` storage,
growth to ``max(needed + reserve, int(1.5 * capacity))`` slots with the old content copied
and unused position slots ``-1`` (cache.py:39-49), ``append`` as two transposing copies plus
the positions (cache.py:51-62), ``view`` as token-major views (cache.py:64-75).  The fused
``append_rotary`` of the kernels is ``append(apply_rotary(k, cos, sin), v, pos)``
(llama.py:161 then cache.py:51-62).  Pinned by known-answer growth sequences and layout
checks in tests/test_oracle_cache.py.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import layers_ref as L


class LayerKVCache:
    def __init__(self, reserve: int = 0) -> None:
        self.k: Optional[torch.Tensor] = None
        self.v: Optional[torch.Tensor] = None
        self.pos: Optional[torch.Tensor] = None
        self.length = 0
        self.reserve = max(0, int(reserve))

    @property
    def capacity(self) -> int:
        return 0 if self.k is None else self.k.shape[2]

    def _grow(self, k, v, pos, needed: int) -> None:  # cache.py:39-49
        capacity = max(needed + self.reserve, int(self.capacity * 1.5))
        B, _, H, D = k.shape
        new_k = k.new_empty((B, H, capacity, D))
        new_v = v.new_empty((B, v.shape[2], capacity, v.shape[3]))
        new_pos = pos.new_full((B, capacity), -1)
        if self.length:
            new_k[:, :, : self.length] = self.k[:, :, : self.length]
            new_v[:, :, : self.length] = self.v[:, :, : self.length]
            new_pos[:, : self.length] = self.pos[:, : self.length]
        self.k, self.v, self.pos = new_k, new_v, new_pos

    def append(self, k, v, pos) -> None:  # cache.py:51-62
        n = k.shape[1]
        if n == 0:
            return
        if self.k is None or self.length + n > self.capacity:
            self._grow(k, v, pos, self.length + n)
        end = self.length + n
        self.k[:, :, self.length: end] = k.transpose(1, 2)
        self.v[:, :, self.length: end] = v.transpose(1, 2)
        self.pos[:, self.length: end] = pos
        self.length = end

    def append_rotary(self, k, v, pos, cos, sin) -> None:
        self.append(L.apply_rotary(k, cos, sin), v, pos)

    def view(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:  # cache.py:64-75
        n = self.length
        return self.k[:, :, :n].transpose(1, 2), self.v[:, :, :n].transpose(1, 2), self.pos[:, :n]
