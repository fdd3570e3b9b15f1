"""The fused column-parallel projections that feed the attention and layer-op kernels,
drop-in for collab_infer/parallel/tensor_parallel.py:264-320 (``FusedColumnParallelLinear``)
and the gate/up half of the gated MLP (collab_infer/models/llama.py:298-316).

Both run on this package's gfx950 GEMM (csrc/gemm.hip): bf16 / f16 on the matrix cores with
f32 accumulation rounded once to the input dtype, f32 / f64 (and shapes the matrix-core
kernel does not take: K or a row stride not a multiple of 8, misaligned rows) on a generic
kernel.

* :func:`linear` - ``F.linear(x, weight, bias)`` for device tensors
* :func:`fused_linear` - the same, returned as the per-projection column views of
  ``.split(local_sizes, dim=-1)`` (tensor_parallel.py:294-295); the rotary, KV-cache append,
  gated-activation and attention kernels take those strided rows as they are
* :func:`linear_gated` - ``act(x.w_gate^T + b_gate) * (x.w_up^T + b_up)`` with the
  reference's rounding points in one pass, so the ``[M, 2I]`` gate/up intermediate never
  reaches memory (llama.py:302-305; the two ``F.linear`` calls of the replicated-token branch,
  llama.py:309-316, are the same call on two row ranges of the fused weight)
* :class:`FusedColumnParallelLinear` - the reference module on one device (its ``comm`` is
  kept for the signature; the local weight is the concatenation of the local slices), with
  :meth:`FusedColumnParallelLinear.gated` for the fused gate/up + activation
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from . import _native as nat
from .layers import ACTIVATION_CODES


def _check_operands(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], what: str):
    if weight.dim() != 2 or x.dim() < 1 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"{what}: x [..., {x.shape[-1] if x.dim() else '?'}] does not match "
                         f"weight {tuple(weight.shape)}")
    if weight.dtype != x.dtype or (bias is not None and bias.dtype != x.dtype):
        raise ValueError(f"{what}: x, weight and bias must share a dtype")
    if bias is not None and tuple(bias.shape) != (weight.shape[0],):
        raise ValueError(f"{what}: bias must be [{weight.shape[0]}], got {tuple(bias.shape)}")


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` for ``x [..., K]``, ``weight [N, K]``, ``bias [N]`` on the
    device; ``out`` may be a preallocated ``[M, N]`` buffer (M = product of x's leading sizes,
    any row stride)."""
    nat.require_device(x, weight, bias, out)
    _check_operands(x, weight, bias, "linear")
    if out is None:
        return nat.ops().linear(x, weight, bias)
    nat.ops().linear_into(out, x, weight, bias)
    return out


def fused_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                 split_sizes: Sequence[int]) -> List[torch.Tensor]:
    """``list(F.linear(x, weight, bias).split(split_sizes, dim=-1))``
    (tensor_parallel.py:294-295)."""
    if sum(split_sizes) != weight.shape[0]:
        raise ValueError(f"split sizes {list(split_sizes)} do not add up to {weight.shape[0]}")
    return list(linear(x, weight, bias).split(list(split_sizes), dim=-1))


def linear_gated(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                 b_gate: Optional[torch.Tensor] = None, b_up: Optional[torch.Tensor] = None,
                 act: str = "silu") -> torch.Tensor:
    """``act(F.linear(x, w_gate, b_gate)) * F.linear(x, w_up, b_up)`` in one pass, with the
    reference's rounding points (each projection and ``act(gate)`` rounded to the dtype before
    the product; llama.py:302-305, 309-316).  ``w_gate`` / ``w_up`` are ``[I, K]`` (e.g. row
    ranges of the fused ``[2I, K]`` parameter), the biases ``[I]`` or both None."""
    nat.require_device(x, w_gate, w_up, b_gate, b_up)
    if act not in ACTIVATION_CODES:
        raise NotImplementedError(f"activation {act!r} is not supported")
    _check_operands(x, w_gate, b_gate, "linear_gated")
    _check_operands(x, w_up, b_up, "linear_gated")
    if w_gate.shape != w_up.shape:
        raise ValueError(f"w_gate {tuple(w_gate.shape)} and w_up {tuple(w_up.shape)} differ")
    if (b_gate is None) != (b_up is None):
        raise ValueError("linear_gated: give both biases or neither")
    return nat.ops().linear_gated(x, w_gate, w_up, b_gate, b_up, ACTIVATION_CODES[act])


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

    def gated(self, x: torch.Tensor, act: str = "silu", units: Optional[Tuple[int, int]] = None) -> torch.Tensor:
        """``act(gate) * up`` of a gate/up layer (two equal parts, gate first) in one pass:
        ``gate, up = self(x); h = act(gate) * up`` (llama.py:302-305).  ``units = (start,
        count)`` restricts it to a slice of the local units, as the replicated-token branch
        does (llama.py:309-316)."""
        if len(self.local_sizes) != 2 or self.local_sizes[0] != self.local_sizes[1]:
            raise ValueError("gated() needs two equal parts: gate and up")
        n = self.local_sizes[0]
        start, count = units if units is not None else (0, n)
        if start < 0 or count < 0 or start + count > n:
            raise ValueError(f"units ({start}, {count}) outside [0, {n})")
        w, b = self.weight, self.bias
        return linear_gated(x, w[start:start + count], w[n + start:n + start + count],
                            None if b is None else b[start:start + count],
                            None if b is None else b[n + start:n + start + count], act)

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


__all__ = ["FusedColumnParallelLinear", "fused_linear", "linear", "linear_gated"]
