"""Pins of the layer-op oracle (oracle/layers_ref.py) on the CPU.

* f64: closed forms written independently of the oracle - RMSNorm per row with numpy
  (the reference's tests/reference.py:17-18), rotary as a complex rotation of the pairs
  (x[i], x[i + D/2]) (half-split, tests/reference.py:21-29), inv_freq = theta^(-2i/D), SiLU as
  g / (1 + exp(-g)); all to 1e-12.
* bf16: the reference rounds at fixed points (llama.py:59-61, 76-77, 87-88, 305).  The
  oracle's bf16 results are compared with the same rounding points applied by an
  independent numpy round-to-nearest-even to the fp64 closed forms: equal except for rare
  last-bit differences of the f32 intermediate (<= 0.5% of elements, never more than one
  bf16 ulp).  A single fused rounding, the classic mistake of a fused kernel, is shown to
  differ in far more elements.
* planted mistakes (interleaved rotary pairs, exponent i/D, missing gate factor, fused
  rounding) are swapped into the oracle and rejected.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import layers_ref as L


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp64 -> f32 -> bf16 (round to nearest even on the upper 16 bits), returned as fp64."""
    f = np.asarray(x, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32).astype(np.float64)


def ulp_bf16(x: np.ndarray) -> np.ndarray:
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---- RMSNorm ------------------------------------------------------------------------------

def _rms_closed(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        row = x[r]
        out[r] = w * (row / math.sqrt(float(np.dot(row, row)) / row.size + eps))
    return out


def test_rmsnorm_f64_closed_form():
    x = torch.randn(64, 256, generator=_gen(0), dtype=torch.float64)
    w = 1 + 0.02 * torch.randn(256, generator=_gen(1), dtype=torch.float64)
    y = L.rmsnorm(x, w, 1e-5).numpy()
    assert np.abs(y - _rms_closed(x.numpy(), w.numpy(), 1e-5)).max() <= 1e-12


def _rms_rounding_points(x, w, eps):
    """bf16(w * bf16(norm)) with norm from the fp64 closed form."""
    xn = x.double().numpy()
    norm = xn / np.sqrt((xn * xn).mean(-1, keepdims=True) + eps)
    return bf16_round(w.double().numpy() * bf16_round(norm))


def test_rmsnorm_bf16_rounding_points():
    x = torch.randn(256, 4096, generator=_gen(2)).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(4096, generator=_gen(3))).to(torch.bfloat16)
    y = L.rmsnorm(x, w, 1e-5).double().numpy()
    want = _rms_rounding_points(x, w, 1e-5)
    diff = np.abs(y - want)
    assert (diff <= ulp_bf16(want) * 1.0001).all()
    assert (diff > 0).mean() <= 5e-3
    # a single rounding of the f32 product misses the reference's intermediate rounding
    xn = x.double().numpy()
    fused = bf16_round(w.double().numpy() * xn / np.sqrt((xn * xn).mean(-1, keepdims=True) + 1e-5))
    assert (fused != want).mean() > 2e-2


def test_planted_fused_rounding_is_caught(monkeypatch):
    def fused(x, weight, eps):
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
        return (weight.float() * h).to(x.dtype)

    monkeypatch.setattr(L, "rmsnorm", fused)
    with pytest.raises(AssertionError):
        test_rmsnorm_bf16_rounding_points()


# ---- rotary ---------------------------------------------------------------------------------

def test_inv_freq_closed_form():
    for D, theta in ((128, 1e4), (64, 5e5), (8, 10.0)):
        inv = L.inv_freq(D, theta).double().numpy()
        want = np.array([theta ** (-2.0 * i / D) for i in range(D // 2)])
        assert np.abs(inv / want - 1).max() <= 2.0 ** -22
        inv64 = L.inv_freq(D, theta, dtype=torch.float64).numpy()
        assert np.abs(inv64 / want - 1).max() <= 1e-14
    lin = L.inv_freq(128, 1e4, {"rope_type": "linear", "factor": 4.0}, dtype=torch.float64).numpy()
    assert np.allclose(lin, L.inv_freq(128, 1e4, dtype=torch.float64).numpy() / 4, rtol=1e-15)


def test_llama3_scaling_regimes():
    """Llama 3.1 frequency scaling: wavelengths below original/high_freq_factor unchanged,
    above original/low_freq_factor divided by factor, smooth and monotone in between."""
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    base = L.inv_freq(128, 5e5, dtype=torch.float64).numpy()
    got = L.inv_freq(128, 5e5, sc, dtype=torch.float64).numpy()
    wl = 2 * math.pi / base
    hi = wl < 8192 / 4.0
    lo = wl > 8192 / 1.0
    assert np.allclose(got[hi], base[hi], rtol=1e-15)
    assert np.allclose(got[lo], base[lo] / 8, rtol=1e-15)
    mid = ~hi & ~lo
    assert mid.any()
    ratio = got[mid] / base[mid]
    assert ((ratio <= 1) & (ratio >= 1 / 8)).all() and (np.diff(ratio) <= 0).all()
    with pytest.raises(NotImplementedError):
        L.inv_freq(128, 1e4, {"rope_type": "yarn", "factor": 2.0})


def _rope_complex(x: np.ndarray, pos: np.ndarray, inv: np.ndarray) -> np.ndarray:
    """x [S, H, D]: pairs (x[i], x[i + D/2]) as complex numbers times exp(i * pos * inv[i])."""
    h = x.shape[-1] // 2
    z = x[..., :h] + 1j * x[..., h:]
    ang = np.maximum(pos, 0)[:, None, None] * inv[None, None, :]
    r = z * np.exp(1j * ang)
    return np.concatenate([r.real, r.imag], axis=-1)


def test_rotary_f64_is_a_rotation_of_half_split_pairs():
    S, H, D = 33, 3, 16
    x = torch.randn(1, S, H, D, generator=_gen(4), dtype=torch.float64)
    pos = torch.arange(S).view(1, S) - 2  # two padding positions clamp to angle 0
    inv = L.inv_freq(D, 1e4, dtype=torch.float64)
    cos, sin = L.rope_tables(pos, inv, torch.float64)
    y = L.apply_rotary(x, cos, sin)[0].numpy()
    want = _rope_complex(x[0].numpy(), pos[0].numpy(), inv.numpy())
    assert np.abs(y - want).max() <= 1e-12
    # norms of the pairs are preserved; padding rows are untouched
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x[0].numpy(), axis=-1))
    assert np.array_equal(y[:3], x[0].numpy()[:3])


def test_planted_interleaved_pairs_are_caught(monkeypatch):
    def interleaved(x):
        out = torch.empty_like(x)
        out[..., 0::2] = -x[..., 1::2]
        out[..., 1::2] = x[..., 0::2]
        return out

    monkeypatch.setattr(L, "rotate_half", interleaved)
    with pytest.raises(AssertionError):
        test_rotary_f64_is_a_rotation_of_half_split_pairs()


def test_planted_exponent_is_caught(monkeypatch):
    good = L.inv_freq

    def wrong(head_dim, theta, scaling=None, dtype=torch.float32):
        return good(2 * head_dim, theta, scaling, dtype)[: head_dim // 2]

    monkeypatch.setattr(L, "inv_freq", wrong)
    with pytest.raises(AssertionError):
        test_inv_freq_closed_form()


def test_rotary_bf16_rounding_points():
    """bf16 tables from f32 angles; x*cos, rot*sin and their sum each rounded to bf16."""
    S, H, D = 512, 4, 128
    x = torch.randn(1, S, H, D, generator=_gen(5)).to(torch.bfloat16)
    pos = torch.arange(S).view(1, S)
    inv = L.inv_freq(D, 1e4)
    cos, sin = L.rope_tables(pos, inv, torch.bfloat16)
    ang = (pos[0].float()[:, None] * inv[None, :]).double().numpy()  # one f32 multiply
    ang = np.concatenate([ang, ang], axis=-1)
    c, s = bf16_round(np.cos(ang)), bf16_round(np.sin(ang))
    assert np.abs(cos[0].double().numpy() - c).max() <= ulp_bf16(c).max()
    assert (cos[0].double().numpy() != c).mean() <= 5e-3
    xn = x[0].double().numpy()
    rot = np.concatenate([-xn[..., D // 2:], xn[..., :D // 2]], axis=-1)
    cc, ss = cos[0].double().numpy()[:, None, :], sin[0].double().numpy()[:, None, :]
    want = bf16_round(bf16_round(xn * cc) + bf16_round(rot * ss))
    y = L.apply_rotary(x, cos, sin)[0].double().numpy()
    assert np.array_equal(y, want)


# ---- SiLU gate ------------------------------------------------------------------------------

def test_silu_gate_f64_closed_form():
    g = torch.randn(64, 300, generator=_gen(6), dtype=torch.float64) * 4
    u = torch.randn(64, 300, generator=_gen(7), dtype=torch.float64)
    gn, un = g.numpy(), u.numpy()
    want = gn / (1 + np.exp(-gn)) * un
    assert np.abs(L.silu_gate(g, u).numpy() - want).max() <= 1e-12


def test_silu_gate_bf16_rounding_points():
    g = torch.randn(512, 1024, generator=_gen(8)).to(torch.bfloat16)
    u = torch.randn(512, 1024, generator=_gen(9)).to(torch.bfloat16)
    gn, un = g.double().numpy(), u.double().numpy()
    want = bf16_round(bf16_round(gn / (1 + np.exp(-gn))) * un)
    y = L.silu_gate(g, u).double().numpy()
    diff = np.abs(y - want)
    assert (diff <= ulp_bf16(want) * 1.0001).all()
    assert (diff > 0).mean() <= 5e-3


def test_planted_missing_gate_factor_is_caught(monkeypatch):
    monkeypatch.setattr(L, "silu_gate", lambda g, u: torch.sigmoid(g) * u)
    with pytest.raises(AssertionError):
        test_silu_gate_f64_closed_form()


# ---- the other gated activations (llama.py:44-49) ---------------------------------------------

_ERF = np.vectorize(math.erf)


def _act_closed(name: str, g: np.ndarray) -> np.ndarray:
    """The activations from their definitions, in f64 (independent of torch)."""
    if name == "silu":
        return g / (1 + np.exp(-g))
    if name == "gelu":  # g * Phi(g), Phi the standard normal CDF
        return g * 0.5 * (1 + _ERF(g / math.sqrt(2.0)))
    if name == "gelu_pytorch_tanh":  # the tanh approximation of Hendrycks & Gimpel (2016)
        return 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
    if name == "relu":
        return np.maximum(g, 0.0)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["silu", "gelu", "gelu_pytorch_tanh", "relu"])
def test_gated_activation_f64_closed_form(name):
    g = torch.randn(64, 300, generator=_gen(16), dtype=torch.float64) * 4
    u = torch.randn(64, 300, generator=_gen(17), dtype=torch.float64)
    want = _act_closed(name, g.numpy()) * u.numpy()
    assert np.abs(L.gated(g, u, name).numpy() - want).max() <= 1e-12


_F32 = np.float32
_ERF32 = np.vectorize(lambda v: _F32(math.erf(float(v))), otypes=[np.float32])
_TANH32 = np.vectorize(lambda v: _F32(math.tanh(float(v))), otypes=[np.float32])


def _act_f32(name: str, g: np.ndarray) -> np.ndarray:
    """The activation formulas evaluated in f32 arithmetic (torch's op math for bf16), with
    correctly rounded erf / tanh; returned as f64."""
    g = g.astype(np.float32)
    if name == "gelu":
        r = (g * _F32(0.5)) * (_F32(1) + _ERF32(g * _F32(0.70710678118654752440)))
    elif name == "gelu_pytorch_tanh":
        inner = _F32(0.79788456080286535588) * (g + _F32(0.044715) * (g * g * g))
        r = (_F32(0.5) * g) * (_F32(1) + _TANH32(inner))
    else:
        r = np.maximum(g, _F32(0))
    return r.astype(np.float64)


@pytest.mark.parametrize("name", ["gelu", "gelu_pytorch_tanh", "relu"])
def test_gated_activation_bf16_rounding_points(name):
    """act(gate) rounded to bf16, then the product rounded (llama.py:305).  The activation
    is computed in f32; where 1 + erf / 1 + tanh cancels (the negative tail) torch's CPU
    erf / tanh differ from correctly rounded ones by up to 2e-5 absolute, scaled by |up|."""
    g = (torch.randn(512, 1024, generator=_gen(18)) * 3).to(torch.bfloat16)
    u = torch.randn(512, 1024, generator=_gen(19)).to(torch.bfloat16)
    gn, un = g.double().numpy(), u.double().numpy()
    want = bf16_round(bf16_round(_act_f32(name, gn)) * un)
    y = L.gated(g, u, name).double().numpy()
    diff = np.abs(y - want)
    assert (diff <= ulp_bf16(want) * 1.0001 + 2e-5 * np.abs(un)).all()
    assert (diff > 0).mean() <= 0.05
    if name == "relu":
        assert (diff == 0).all()
    # a single fused rounding of act * up misses the first rounding point in many elements
    fused = bf16_round(_act_f32(name, gn) * un)
    if name != "relu":
        assert (np.abs(fused - want) > 0).mean() > 0.05


def test_gelu_planted_mistakes_are_caught(monkeypatch):
    """The two GELU forms differ by up to ~5e-4, far above the f64 pins: swapping them, or
    dropping the cubic term of the tanh form, fails the closed-form check."""
    tanh_form = L.ACTIVATIONS["gelu_pytorch_tanh"]
    monkeypatch.setitem(L.ACTIVATIONS, "gelu", tanh_form)
    with pytest.raises(AssertionError):
        test_gated_activation_f64_closed_form("gelu")
    monkeypatch.setitem(L.ACTIVATIONS, "gelu_pytorch_tanh",
                        lambda x: 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * x)))
    with pytest.raises(AssertionError):
        test_gated_activation_f64_closed_form("gelu_pytorch_tanh")


def test_rmsnorm_rope_f64_composition():
    S, H, D = 17, 4, 32
    x = torch.randn(S, H * D, generator=_gen(10), dtype=torch.float64)
    w = 1 + 0.02 * torch.randn(H * D, generator=_gen(11), dtype=torch.float64)
    pos = torch.arange(S)
    inv = L.inv_freq(D, 1e4, dtype=torch.float64)
    y = L.rmsnorm_rope(x, w, 1e-5, pos, inv, H)[0].numpy()
    normed = _rms_closed(x.numpy(), w.numpy(), 1e-5).reshape(S, H, D)
    want = _rope_complex(normed, pos.numpy(), inv.numpy())
    assert np.abs(y - want).max() <= 1e-12


# ---- fused projection (tensor_parallel.py:294-295) -----------------------------------------

def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (2^(e-7) for |x| in [2^e, 2^(e+1)))."""
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -126)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("bias", [False, True])
def test_oracle_linear_closed_form(bias):
    """The oracle's projection equals x . W^T + b computed in f64, to the output rounding (bf16:
    within one bf16 ulp of the f64 value plus the f32 accumulation error); a transposed
    weight or a dropped bias is rejected by the same check."""
    g = torch.Generator().manual_seed(3)
    N, K, M = 37, 256, 256
    x = torch.randn(N, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(M, K, generator=g) / 16).to(torch.bfloat16)
    b = torch.randn(M, generator=g).to(torch.bfloat16) if bias else None
    exact = x.double() @ w.double().T + (b.double() if bias else 0)

    def close(y):
        err = (y.double() - exact).abs()
        return bool((err <= _bf16_ulp(exact) + 1e-4 * exact.abs().max()).all())

    assert close(L.linear(x, w, b))
    assert not close(L.linear(x, w.T.contiguous(), b))
    if bias:
        assert not close(L.linear(x, w, None))


# ---------------------------------------------------------------------------------------
# linear (tensor_parallel.py:294-295): F.linear in the input dtype on the CPU
# ---------------------------------------------------------------------------------------
def _exact_linear(x, w, b):
    y = x.double() @ w.double().t()
    return y if b is None else y + b.double()


def test_linear_f64_closed_form():
    """y[i, j] = sum_k x[i, k] w[j, k] + b[j]: integer-valued operands make every product and
    sum exact, so the oracle must return the exact integers (a transposed weight, a dropped
    bias or a wrong contraction axis changes them)."""
    g = torch.Generator().manual_seed(4)
    x = torch.randint(-8, 9, (5, 7), generator=g).double()
    w = torch.randint(-8, 9, (3, 7), generator=g).double()
    b = torch.randint(-8, 9, (3,), generator=g).double()
    want = torch.tensor([[sum(x[i, k].item() * w[j, k].item() for k in range(7)) + b[j].item()
                          for j in range(3)] for i in range(5)], dtype=torch.float64)
    assert torch.equal(L.linear(x, w, b), want)
    assert torch.equal(L.linear(x, w), want - b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_reduced_precision_rounds_once(dtype):
    """bf16 / f16 F.linear accumulates in f32 and rounds once: within the f32 accumulation
    bound of the exact result, and equal to the correctly rounded exact value for almost
    every element (a per-term rounding to the dtype would break both)."""
    g = torch.Generator().manual_seed(5)
    m, k, n = 64, 1024, 96
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) / 32).to(dtype)
    b = torch.randn(n, generator=g).to(dtype)
    y = L.linear(x, w, b)
    exact = _exact_linear(x, w, b)
    mags = x.double().abs() @ w.double().abs().t() + b.double().abs()
    gam = (k + 2) * 2.0 ** -24 * mags
    mant = 7 if dtype == torch.bfloat16 else 10
    e = torch.floor(torch.log2((exact.abs() + gam).clamp(min=2.0 ** -30)))
    ulp = torch.pow(2.0, e - mant)
    assert bool(((y.double() - exact).abs() <= ulp / 2 + gam).all())
    assert (y == exact.to(dtype)).double().mean().item() >= 0.99
