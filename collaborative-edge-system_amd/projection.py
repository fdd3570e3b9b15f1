"""The fused Q/K/V and gate/up projections that feed the attention and layer-op kernels,
drop-in for collab_infer/parallel/tensor_parallel.py:264-320 (``FusedColumnParallelLinear``).

The projection itself is a plain library GEMM: it stays the reference's ``F.linear``, run by
PyTorch's own BLAS on the device (this package ships no GEMM kernel and links no BLAS
library of its own, so it never mixes a second BLAS build into the process).  What this
module adds is the layout contract: the per-projection outputs are column views of the one
GEMM output, and the rotary, KV-cache append, SiLU-gate and attention kernels take those
strided rows as they are, without a copy.

* :func:`linear` - ``F.linear(x, weight, bias)`` for device tensors
* :func:`fused_linear` - the same, returned as the per-projection column views of
  ``.split(local_sizes, dim=-1)``
* :class:`FusedColumnParallelLinear` - the reference module on one device (its ``comm`` is
  kept for the signature; the local weight is the concatenation of the local slices)
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as nat


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` for ``x [..., K]``, ``weight [M, K]``, ``bias [M]`` on the
    device; ``out`` may be a preallocated ``[N, M]`` buffer (N = product of x's leading sizes)."""
    nat.require_device(x, weight, bias, out)
    if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"linear: x [..., {x.shape[-1]}] does not match weight {tuple(weight.shape)}")
    if weight.dtype != x.dtype or (bias is not None and bias.dtype != x.dtype):
        raise ValueError("linear: x, weight and bias must share a dtype")
    y = F.linear(x, weight, bias)
    if out is None:
        return y
    out.copy_(y.reshape(-1, weight.shape[0]))
    return out


def fused_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                 split_sizes: Sequence[int]) -> List[torch.Tensor]:
    """``list(F.linear(x, weight, bias).split(split_sizes, dim=-1))``
    (tensor_parallel.py:294-295)."""
    if sum(split_sizes) != weight.shape[0]:
        raise ValueError(f"split sizes {list(split_sizes)} do not add up to {weight.shape[0]}")
    return list(linear(x, weight, bias).split(list(split_sizes), dim=-1))


class FusedColumnParallelLinear(nn.Module):
    """Several column-parallel projections of one input computed by one GEMM
    (tensor_parallel.py:264-313).  ``parts`` lists ``(out_features, local_start, local_size)``
    per projection; :meth:`forward` returns the per-projection outputs."""

    def __init__(self, in_features: int, parts: Sequence[Tuple[int, int, int]], comm=None, *,
                 bias: bool = False, dtype: Optional[torch.dtype] = None,
                 device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.comm = comm
        self.in_features = in_features
        self.parts = [(int(o), int(s), int(n)) for o, s, n in parts]
        for out, start, size in self.parts:
            if start < 0 or size < 0 or start + size > out:
                raise ValueError(f"local range ({start}, {size}) outside [0, {out})")
        self.local_sizes = [n for _, _, n in self.parts]
        total = sum(self.local_sizes)
        self.weight = nn.Parameter(torch.empty(total, in_features, dtype=dtype, device=device),
                                   requires_grad=False)
        self.bias = (nn.Parameter(torch.empty(total, dtype=dtype, device=device), requires_grad=False)
                     if bias else None)

    def forward(self, x: torch.Tensor) -> List[torch.Tensor]:
        return fused_linear(x, self.weight, self.bias, self.local_sizes)

    @torch.no_grad()
    def load_full(self, weights: Sequence[torch.Tensor],
                  biases: Optional[Sequence[Optional[torch.Tensor]]] = None) -> None:
        """Load from the full (unsharded) parameters of every fused projection."""
        if len(weights) != len(self.parts):
            raise ValueError(f"expected {len(self.parts)} weights, got {len(weights)}")
        offset = 0
        for i, (_, start, size) in enumerate(self.parts):
            src = weights[i].narrow(0, start, size)
            dst = self.weight[offset:offset + size]
            if tuple(dst.shape) != tuple(src.shape):
                raise ValueError(f"shape mismatch: parameter {tuple(dst.shape)} vs value {tuple(src.shape)}")
            dst.copy_(src.to(dtype=dst.dtype, device=dst.device))
            if self.bias is not None:
                if biases is None or biases[i] is None:
                    raise ValueError("layer has a bias but none was provided")
                self.bias[offset:offset + size].copy_(
                    biases[i].narrow(0, start, size).to(dtype=self.bias.dtype, device=self.bias.device))
            offset += size

    def extra_repr(self) -> str:
        return f"in={self.in_features}, parts={self.parts}, bias={self.bias is not None}"


__all__ = ["FusedColumnParallelLinear", "fused_linear", "linear"]
