"""CPU restatement of the LLaMA layer ops with the reference's rounding points (test
infrastructure only).

Each function runs the same sequence of separately rounded torch CPU ops as the reference,
so in bf16 it defines the expected bits of the fused kernels (up to the last bit of the
transcendental functions, whose implementations differ between CPU and GPU math libraries).
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """llama.py:58-61: f32 (f64 for f64) normalisation, rounded to x.dtype, times weight."""
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    h = x.to(acc)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)


def inv_freq(head_dim: int, theta: float, scaling: Optional[dict] = None,
             dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """models/config.py:165-189 (``rope_inv_freq``)."""
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
        lo, hi = scaling["low_freq_factor"], scaling["high_freq_factor"]
        old = scaling["original_max_position_embeddings"]
        wl = 2 * math.pi / inv
        scaled = torch.where(wl > old / lo, inv / factor, inv)
        sm = (old / wl - lo) / (hi - lo)
        smoothed = (1 - sm) * scaled / factor + sm * scaled
        medium = ~(wl < old / hi) & ~(wl > old / lo)
        return torch.where(medium, smoothed, scaled)
    raise NotImplementedError(f"rope scaling type {kind!r} is not supported")


def rope_tables(positions: torch.Tensor, inv: torch.Tensor, dtype: torch.dtype):
    """llama.py:74-77: clamp(pos, 0) * inv_freq, duplicated halves, cos/sin to dtype."""
    pos = positions.clamp(min=0).to(inv.dtype)
    freqs = pos.unsqueeze(-1) * inv
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """llama.py:80-82."""
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """llama.py:85-88: x [B,S,H,D], tables [B,S,D]."""
    return x * cos.unsqueeze(2) + rotate_half(x) * sin.unsqueeze(2)


def rmsnorm_rope(x, weight, eps, positions, inv, num_heads):
    """RMSNorm of x [S, C], viewed [1, S, H, D], rotated at positions [1, S]."""
    y = rmsnorm(x, weight, eps)
    S, C = y.shape
    y = y.view(1, S, num_heads, C // num_heads)
    cos, sin = rope_tables(positions.view(1, S), inv, x.dtype)
    return apply_rotary(y, cos, sin)


def silu_gate(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """llama.py:45, 305: F.silu(gate) * up."""
    return F.silu(gate) * up


# llama.py:44-49 (_ACTIVATIONS)
ACTIVATIONS = {
    "silu": F.silu,
    "gelu": F.gelu,
    "gelu_pytorch_tanh": lambda x: F.gelu(x, approximate="tanh"),
    "relu": F.relu,
}


def gated(gate: torch.Tensor, up: torch.Tensor, act: str) -> torch.Tensor:
    """llama.py:305: self.act(gate) * up, two separately rounded tensor ops."""
    return ACTIVATIONS[act](gate) * up


def linear(x, weight, bias=None):
    """tensor_parallel.py:294-295: F.linear of the fused projection, in the input dtype on the
    CPU (f32 accumulation for bf16 / f16 inputs)."""
    return torch.nn.functional.linear(x, weight, bias)
