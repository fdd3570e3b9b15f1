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

import itertools
from typing import List, NamedTuple, Optional, Sequence, Tuple

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


class _Slice(NamedTuple):
    """One projection of a fused layer: its full width ``full``, the rows ``[start, start +
    size)`` of it this rank holds, and the first row ``row0`` of those in the fused weight."""

    full: int
    start: int
    size: int
    row0: int


def _slices(parts: Sequence[Tuple[int, int, int]]) -> List[_Slice]:
    """The fused weight's row layout: local slices stacked in part order.  Raises ValueError
    naming every part whose local range leaves ``[0, out_features)``."""
    triples = [tuple(int(v) for v in t) for t in parts]
    bad = [f"part {i}: ({s}, {n}) outside [0, {o})" for i, (o, s, n) in enumerate(triples)
           if s < 0 or n < 0 or s + n > o]
    if bad:
        raise ValueError("local range outside the projection: " + "; ".join(bad))
    starts = itertools.accumulate((n for _, _, n in triples), initial=0)
    return [_Slice(o, s, n, r) for (o, s, n), r in zip(triples, starts)]


class FusedColumnParallelLinear(nn.Module):
    """Several column-parallel projections of one input computed by one GEMM
    (tensor_parallel.py:264-313).  ``parts`` lists ``(out_features, local_start, local_size)``
    per projection; :meth:`forward` returns the per-projection outputs as column views of
    the one GEMM result."""

    def __init__(self, in_features: int, parts: Sequence[Tuple[int, int, int]], comm=None, *,
                 bias: bool = False, dtype: Optional[torch.dtype] = None,
                 device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.comm = comm
        self.in_features = int(in_features)
        self._slices = _slices(parts)
        rows = sum(sl.size for sl in self._slices)
        make = lambda *shape: nn.Parameter(torch.empty(*shape, dtype=dtype, device=device),
                                           requires_grad=False)
        self.weight = make(rows, self.in_features)
        self.bias = make(rows) if bias else None

    @property
    def parts(self) -> List[Tuple[int, int, int]]:
        return [(sl.full, sl.start, sl.size) for sl in self._slices]

    @property
    def local_sizes(self) -> List[int]:
        return [sl.size for sl in self._slices]

    def forward(self, x: torch.Tensor) -> List[torch.Tensor]:
        return fused_linear(x, self.weight, self.bias, self.local_sizes)

    def gated(self, x: torch.Tensor, act: str = "silu", units: Optional[Tuple[int, int]] = None) -> torch.Tensor:
        """``act(gate) * up`` of a gate/up layer (two equal parts, gate first) in one pass:
        ``gate, up = self(x); h = act(gate) * up`` (llama.py:302-305).  ``units = (start,
        count)`` restricts it to a slice of the local units, as the replicated-token branch
        does (llama.py:309-316)."""
        if len(self._slices) != 2 or self._slices[0].size != self._slices[1].size:
            raise ValueError("gated() needs two equal parts: gate and up")
        gate, up = self._slices
        start, count = units if units is not None else (0, gate.size)
        if start < 0 or count < 0 or start + count > gate.size:
            raise ValueError(f"units ({start}, {count}) outside [0, {gate.size})")
        rows_g = slice(gate.row0 + start, gate.row0 + start + count)
        rows_u = slice(up.row0 + start, up.row0 + start + count)
        w, b = self.weight, self.bias
        return linear_gated(x, w[rows_g], w[rows_u], None if b is None else b[rows_g],
                            None if b is None else b[rows_u], act)

    @torch.no_grad()
    def load_full(self, weights: Sequence[torch.Tensor],
                  biases: Optional[Sequence[Optional[torch.Tensor]]] = None) -> None:
        """Fill the fused parameters from the full (unsharded) parameters of every projection:
        this rank's rows of each, stacked in part order, copied in one go."""
        if len(weights) != len(self._slices):
            raise ValueError(f"expected {len(self._slices)} weights, got {len(weights)}")
        if self.bias is not None and (biases is None or len(biases) != len(self._slices)
                                      or any(t is None for t in biases)):
            raise ValueError("layer has a bias but none was provided")

        def stacked(full: Sequence[torch.Tensor], param: torch.Tensor) -> torch.Tensor:
            rows = [t.narrow(0, sl.start, sl.size).to(param.device, param.dtype)
                    for t, sl in zip(full, self._slices)]
            got = torch.cat(rows, 0)
            if got.shape != param.shape:
                raise ValueError(f"shape mismatch: parameter {tuple(param.shape)} vs value {tuple(got.shape)}")
            return got

        self.weight.copy_(stacked(weights, self.weight))
        if self.bias is not None:
            self.bias.copy_(stacked(biases, self.bias))

    def extra_repr(self) -> str:
        layout = ", ".join(f"{sl.size} of {sl.full} from {sl.start}" for sl in self._slices)
        return (f"in_features={self.in_features}, rows={self.weight.shape[0]} ({layout}), "
                f"bias={self.bias is not None}")


__all__ = ["FusedColumnParallelLinear", "fused_linear", "linear", "linear_gated"]
