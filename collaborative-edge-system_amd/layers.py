"""LLaMA / Mistral / Qwen2 layer ops on MI355X, drop-in for the calls in
collab_infer/models/llama.py.

* :class:`RMSNorm` - llama.py:52-61 (``weight * (x * rsqrt(mean(x^2) + eps)).to(x.dtype)``)
* :class:`RotaryEmbedding` - llama.py:64-77 (cos/sin at explicit positions, computed once per
  pass), with :func:`rope_inv_freq` from models/config.py:165-189
* :func:`apply_rotary` - llama.py:80-88 (half-split rotation)
* :func:`gated_mul` / :func:`silu_mul` - ``act(gate) * up`` for every activation of the
  reference's ``_ACTIVATIONS`` (silu, gelu, gelu_pytorch_tanh, relu; llama.py:44-49, 305, 316)
* :func:`rmsnorm_rope` - RMSNorm, rotary tables and rotation fused into one pass

Each kernel reproduces the rounding points of the reference's separate tensor ops, so in
bf16 the fused kernels return what the op sequence returns (up to the last bit of the
transcendental functions).
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from . import _native as nat


def rope_inv_freq(head_dim: int, theta: float, scaling: Optional[dict] = None,
                  dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Inverse rotary frequencies ``1 / theta^(2i/D)`` with ``linear`` / ``llama3`` scaling
    (models/config.py:165-189).  Configuration-time host arithmetic on a ``D/2`` vector."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).to(dtype) / head_dim
    inv = 1.0 / (theta ** exponent)
    if not scaling:
        return inv
    kind = scaling.get("rope_type", scaling.get("type", "default"))
    if kind == "default":
        return inv
    if kind == "linear":
        return inv / scaling["factor"]
    if kind == "llama3":
        factor = scaling["factor"]
        lo_f, hi_f = scaling["low_freq_factor"], scaling["high_freq_factor"]
        ctx = scaling["original_max_position_embeddings"]
        lo_wave, hi_wave = ctx / lo_f, ctx / hi_f
        wave = 2 * math.pi / inv
        scaled = torch.where(wave > lo_wave, inv / factor, inv)
        t = (ctx / wave - lo_f) / (hi_f - lo_f)
        blended = (1 - t) * scaled / factor + t * scaled
        mid = ~(wave < hi_wave) & ~(wave > lo_wave)
        return torch.where(mid, blended, scaled)
    raise NotImplementedError(f"rope scaling type {kind!r} is not supported")


def _rows(x: torch.Tensor) -> torch.Tensor:
    """``[..., C]`` as a 2-D ``[N, C]`` view (copying only if the rows cannot be strided)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    try:
        return x.view(-1, x.shape[-1])
    except RuntimeError:
        return x.reshape(-1, x.shape[-1])


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Functional RMSNorm with the reference's rounding (llama.py:58-61)."""
    return nat.ops().rmsnorm(_rows(x), weight, float(eps)).view(x.shape)


class RMSNorm(nn.Module):
    """RMSNorm module (llama.py:52-61)."""

    def __init__(self, dim: int, eps: float, dtype=None, device=None) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype, device=device), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rmsnorm(x, self.weight, self.eps)


def rope_tables(positions: torch.Tensor, inv_freq: torch.Tensor, dtype: torch.dtype):
    """``(cos, sin)`` tables ``[B, S, D]`` in ``dtype`` at explicit positions (llama.py:74-77)."""
    pos = positions.unsqueeze(0) if positions.dim() == 1 else positions
    want = torch.float64 if dtype == torch.float64 else torch.float32
    cos, sin = nat.ops().rope_tables(pos, inv_freq.to(want).contiguous(), dtype)
    return cos, sin


class RotaryEmbedding(nn.Module):
    """Rotary position embedding evaluated at explicit positions (llama.py:64-77).

    ``config`` needs ``head_dim``, ``rope_theta`` and optionally ``rope_scaling`` (the
    fields of collab_infer's ``ModelConfig``).
    """

    def __init__(self, config, device=None) -> None:
        super().__init__()
        scaling = getattr(config, "rope_scaling", None)
        self.register_buffer(
            "inv_freq32", rope_inv_freq(config.head_dim, config.rope_theta, scaling, torch.float32).to(device),
            persistent=False)
        self.register_buffer(
            "inv_freq64", rope_inv_freq(config.head_dim, config.rope_theta, scaling, torch.float64).to(device),
            persistent=False)

    def forward(self, positions: torch.Tensor, dtype: torch.dtype):
        inv = self.inv_freq64 if dtype == torch.float64 else self.inv_freq32
        return rope_tables(positions, inv, dtype)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x``: ``[B, S, H, D]``; ``cos``/``sin``: ``[B, S, D]`` (llama.py:85-88)."""
    if cos.dtype != x.dtype or sin.dtype != x.dtype:
        # the reference multiplies in the promoted dtype; tables in the model dtype are the
        # convention of RotaryEmbedding, other combinations are converted explicitly
        cos, sin = cos.to(x.dtype), sin.to(x.dtype)
    return nat.ops().apply_rotary(x, cos, sin)


def rmsnorm_rope(x: torch.Tensor, weight: torch.Tensor, eps: float, positions: torch.Tensor,
                 inv_freq: torch.Tensor, num_heads: int) -> torch.Tensor:
    """RMSNorm of ``x`` ``[S, H*D]`` followed by rotary at ``positions`` ``[S]`` on the
    ``[1, S, H, D]`` view, in one kernel.  Returns ``[1, S, H, D]``."""
    x2 = _rows(x)
    S, C = x2.shape
    if C % num_heads:
        raise ValueError(f"{C} features do not split into {num_heads} heads")
    want = torch.float64 if x.dtype == torch.float64 else torch.float32
    out = nat.ops().rmsnorm_rope(x2, weight, float(eps), positions.reshape(-1),
                                 inv_freq.to(want).contiguous(), int(num_heads))
    return out.view(1, S, num_heads, C // num_heads)


# the reference's activation names (llama.py:44-49) -> CEA_ACT_* codes of cea_gated_mul
ACTIVATION_CODES = {"silu": 0, "gelu": 1, "gelu_pytorch_tanh": 2, "relu": 3}


def gated_mul(gate: torch.Tensor, up: torch.Tensor, act: str = "silu") -> torch.Tensor:
    """``act(gate) * up`` (llama.py:44-49, 305) with ``act`` one of the reference's
    activations; ``gate``/``up`` may be column halves of one fused GEMM output."""
    if act not in ACTIVATION_CODES:
        raise NotImplementedError(f"activation {act!r} is not supported")
    if gate.shape != up.shape:
        raise ValueError(f"gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
    return nat.ops().gated_mul(_rows(gate), _rows(up), ACTIVATION_CODES[act]).view(gate.shape)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate) * up`` (llama.py:305)."""
    return gated_mul(gate, up, "silu")


class _GatedActivation:
    """``act(gate) * up`` for one activation name, as one kernel."""

    def __init__(self, name: str) -> None:
        self.name = name

    def __call__(self, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        return gated_mul(gate, up, self.name)

    def __repr__(self) -> str:
        return f"gated_activation({self.name!r})"


def gated_activation(name: str):
    """The fused ``act(gate) * up`` for a model's ``hidden_act`` (llama.py:44-49, 298)."""
    if name not in ACTIVATION_CODES:
        raise NotImplementedError(f"activation {name!r} is not supported")
    return _GatedActivation(name)


__all__ = [
    "ACTIVATION_CODES",
    "RMSNorm",
    "RotaryEmbedding",
    "apply_rotary",
    "gated_activation",
    "gated_mul",
    "rmsnorm",
    "rmsnorm_rope",
    "rope_inv_freq",
    "rope_tables",
    "silu_mul",
]
