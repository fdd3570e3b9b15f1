"""GPU parity of the layer-op kernels (RMSNorm, rotary tables, rotary, fused RMSNorm+rotary,
SiLU gate) against the CPU oracle, through the C ABI.

Tolerances (written here, used below):
* bf16 and f16: every element within one ulp of its dtype of the oracle (the oracle rounds at the
  reference's points, so only a last-bit difference of a transcendental or an f32
  intermediate can remain), at most 1e-3 of the elements differing at all, and
  max |diff| <= 2e-2 over elements with |ref| < 2 (the workload's absolute bound; above 2 a
  single bf16 ulp is larger than 2e-2, and the ulp bound applies).  For RMSNorm followed by
  rotary, a last-bit flip of the normalised value y propagates through x*cos + rot*sin,
  whose sum may be much smaller than its terms: there the bound is two ulps of the larger
  term magnitude max(|y_i|, |y_j|) of the rotated pair, with the same 1e-3 and 2e-2 rules
  on that magnitude;
* f32: normwise rel <= 1e-6;  f64: max abs <= 1e-12.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import layers_ref as L

pytestmark = pytest.mark.gpu


def _ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Spacing of ``dtype`` (bf16 or f16) at magnitude |x|."""
    mant, emin = (7, -126) if dtype == torch.bfloat16 else (10, -14)
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** emin)))
    return torch.exp2(e - mant)


def assert_close_layer(y: torch.Tensor, ref: torch.Tensor, what: str, mag: torch.Tensor = None,
                       ulps: float = 1.0):
    """``mag``: magnitude the bf16 ulp bound is taken from (default |ref|)."""
    y = y.detach().cpu()
    assert y.shape == ref.shape and y.dtype == ref.dtype, (what, y.shape, ref.shape, y.dtype, ref.dtype)
    if y.dtype == torch.float64:
        err = (y - ref).abs().max().item()
        assert err <= 1e-12, f"{what}: {err:.3e}"
        return
    if y.dtype == torch.float32:
        err = (y - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
        assert err <= 1e-6, f"{what}: rel {err:.3e}"
        return
    a, b = y.float(), ref.float()
    m = b.abs() if mag is None else mag.float().abs()
    diff = (a - b).abs()
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    over = diff > _ulp(m, y.dtype) * ulps * 1.0001
    assert not over.any(), f"{what}: {int(over.sum())} elements beyond {ulps} ulp, max {diff.max().item():.3e}"
    frac = (diff > 0).float().mean().item()
    assert frac <= 1e-3, f"{what}: {frac:.2e} of the elements differ"
    small = m < 2
    if small.any():
        assert diff[small].max().item() <= 2e-2, what


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (4096, 4096)), (torch.float32, (64, 1000)),
                                         (torch.float64, (8, 300)), (torch.float16, (33, 512))])
def test_rmsnorm(cea, dev, dtype, shape):
    x = torch.randn(*shape, generator=_gen(0)).to(dtype)
    w = (1 + 0.02 * torch.randn(shape[-1], generator=_gen(1))).to(dtype)
    y = cea.layers.rmsnorm(x.to(dev), w.to(dev), 1e-5)
    torch.cuda.synchronize()
    assert_close_layer(y, L.rmsnorm(x, w, 1e-5), f"rmsnorm {dtype}")


def test_rmsnorm_module_mixed_dtypes_and_views(cea, dev):
    """A f32 weight on bf16 activations promotes (llama.py:61); non-contiguous rows."""
    x = torch.randn(3, 40, 256, generator=_gen(2)).to(torch.bfloat16)
    w = 1 + 0.02 * torch.randn(256, generator=_gen(3))
    y = cea.layers.rmsnorm(x.to(dev), w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert_close_layer(y, L.rmsnorm(x, w, 1e-6), "rmsnorm promoted")
    big = torch.randn(40, 512, generator=_gen(4)).to(torch.bfloat16)
    view = big[:, 128:384]  # row stride 512
    m = cea.RMSNorm(256, 1e-5, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    assert_close_layer(m(view.to(dev)), L.rmsnorm(view, torch.ones(256, dtype=torch.bfloat16), 1e-5),
                       "rmsnorm view")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
def test_rope_tables_and_rotary(cea, dev, dtype):
    S, H, D = 4096, 32, 128
    pos = torch.arange(S).view(1, S)
    pos[0, :5] = -1  # padding: angle 0
    inv = L.inv_freq(D, 1e4, dtype=torch.float64 if dtype == torch.float64 else torch.float32)
    cos, sin = cea.layers.rope_tables(pos.to(dev), inv.to(dev), dtype)
    rc, rs = L.rope_tables(pos, inv, dtype)
    x = torch.randn(1, S, H, D, generator=_gen(5)).to(dtype)
    y = cea.layers.apply_rotary(x.to(dev), cos, sin)
    torch.cuda.synchronize()
    assert_close_layer(cos, rc, "cos")
    assert_close_layer(sin, rs, "sin")
    # rotary on the kernel's own tables vs the oracle on the same tables
    assert_close_layer(y, L.apply_rotary(x, cos.cpu(), sin.cpu()), "apply_rotary")


def test_rotary_embedding_module_llama3_scaling(cea, dev):
    cfg = SimpleNamespace(head_dim=64, rope_theta=5e5,
                          rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                        "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    rot = cea.RotaryEmbedding(cfg, device=dev)
    pos = torch.arange(0, 20000, 7).view(1, -1)
    cos, sin = rot(pos.to(dev), torch.float32)
    inv = L.inv_freq(64, 5e5, cfg.rope_scaling)
    rc, rs = L.rope_tables(pos, inv, torch.float32)
    torch.cuda.synchronize()
    # f32 tables: the angle is one f32 multiply in both; cos/sin of large angles differ by
    # the f32 rounding of the argument reduction, bounded here absolutely
    assert (cos.cpu() - rc).abs().max().item() <= 2e-6
    assert (sin.cpu() - rs).abs().max().item() <= 2e-6


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rmsnorm_rope_fused(cea, dev, dtype):
    """RMSNorm [4096, 4096] then rotary on the [1, 4096, 32, 128] view at positions 0..4095."""
    S, H, D = 4096, 32, 128
    x = torch.randn(S, H * D, generator=_gen(6)).to(dtype)
    w = (1 + 0.02 * torch.randn(H * D, generator=_gen(7))).to(dtype)
    pos = torch.arange(S)
    inv = L.inv_freq(D, 1e4)
    y = cea.rmsnorm_rope(x.to(dev), w.to(dev), 1e-5, pos.to(dev), inv.to(dev), H)
    torch.cuda.synchronize()
    normed = L.rmsnorm(x, w, 1e-5).view(1, S, H, D).float()
    pair = torch.maximum(normed.abs(), L.rotate_half(normed).abs())
    assert_close_layer(y, L.rmsnorm_rope(x, w, 1e-5, pos, inv, H), f"rmsnorm_rope {dtype}",
                       mag=pair, ulps=2.0)


@pytest.mark.parametrize("S,H,D,dtype", [
    (7, 3, 64, torch.bfloat16),      # odd row count, 12 of 256 threads own a chunk
    (5, 8, 512, torch.float16),      # D/2 = 256: the largest single-pass table
    (3, 2, 1024, torch.bfloat16),    # D/2 = 512: the two-pass kernel
    (9, 64, 128, torch.bfloat16),    # 512 chunks per row: the two-pass kernel
    (6, 4, 96, torch.float32),       # 4-wide f32 chunks
])
def test_rmsnorm_rope_shapes(cea, dev, S, H, D, dtype):
    """Row counts that leave a partial block, rows with idle threads, both kernels, a
    row-strided input view and negative (clamped) positions."""
    base = torch.randn(S, H * D + 64, generator=_gen(11)).to(dtype)
    x = base[:, :H * D]  # row stride H*D + 64
    w = (1 + 0.05 * torch.randn(H * D, generator=_gen(12))).to(dtype)
    pos = torch.randint(-3, 5000, (S,), generator=_gen(13))
    inv = L.inv_freq(D, 1e4)
    y = cea.rmsnorm_rope(base.to(dev)[:, :H * D], w.to(dev), 1e-6, pos.to(dev), inv.to(dev), H)
    torch.cuda.synchronize()
    normed = L.rmsnorm(x, w, 1e-6).view(1, S, H, D).float()
    pair = torch.maximum(normed.abs(), L.rotate_half(normed).abs())
    ref = L.rmsnorm_rope(x, w, 1e-6, pos, inv, H)
    if dtype == torch.float32:
        assert (y.cpu() - ref).abs().max().item() <= 1e-5 * max(1.0, ref.abs().max().item())
    else:
        assert_close_layer(y, ref, f"rmsnorm_rope {S}x{H}x{D} {dtype}", mag=pair, ulps=2.0)


@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (4096, 14336)), (torch.float32, (100, 3000)),
                                         (torch.float64, (10, 77)), (torch.bfloat16, (70000, 24)),
                                         (torch.float16, (3, 2056))])
def test_silu_mul(cea, dev, dtype, shape):
    g = torch.randn(*shape, generator=_gen(8)).to(dtype)
    u = torch.randn(*shape, generator=_gen(9)).to(dtype)
    y = cea.silu_mul(g.to(dev), u.to(dev))
    torch.cuda.synchronize()
    assert_close_layer(y, L.silu_gate(g, u), f"silu_mul {dtype}")


def test_silu_mul_on_fused_gemm_halves(cea, dev):
    """gate/up as column halves of one [T, 2I] GEMM output (row stride 2I)."""
    fused = torch.randn(512, 2 * 1000, generator=_gen(10)).to(torch.bfloat16)
    g, u = fused[:, :1000], fused[:, 1000:]
    fd = fused.to(dev)
    y = cea.layers.gated_activation("silu")(fd[:, :1000], fd[:, 1000:])
    torch.cuda.synchronize()
    assert_close_layer(y, L.silu_gate(g, u), "silu halves")


@pytest.mark.parametrize("act", ["gelu", "gelu_pytorch_tanh", "relu"])
@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (4096, 14336)), (torch.float16, (300, 2056)),
                                         (torch.float32, (100, 3000)), (torch.float64, (10, 77))])
def test_gated_activations(cea, dev, act, dtype, shape):
    """gelu / gelu_pytorch_tanh / relu gates (llama.py:44-49, 305) against the oracle's
    separately rounded torch ops; gate values spread over +-8 so the activations' tails and
    the relu kink are exercised."""
    g = (torch.randn(*shape, generator=_gen(20)) * 3).to(dtype)
    u = torch.randn(*shape, generator=_gen(21)).to(dtype)
    y = cea.layers.gated_mul(g.to(dev), u.to(dev), act)
    y2 = cea.layers.gated_activation(act)(g.to(dev), u.to(dev))
    torch.cuda.synchronize()
    ref = L.gated(g, u, act)
    assert torch.equal(y, y2)
    if act == "relu" or dtype == torch.float64:
        assert_close_layer(y, ref, f"{act} {dtype}")
        return
    # Both sides evaluate the GELU forms in f32 with different erf / tanh implementations
    # (torch's vectorised CPU code differs from correctly rounded values in a third of the
    # elements, by up to 1e-6 absolute and, in the negative tail where 1 + erf(x/sqrt 2) and
    # 1 + tanh(.) cancel, 2e-5).  f32: the north-star tolerance, normwise rel <= 1e-5.  bf16 /
    # f16: a last-bit flip of the rounded activation reaches the result scaled by |up|, so the
    # bound is one ulp of the result + one ulp of the activation times |up| + 2e-5 |up|, and
    # the abs bound 2e-2 holds wherever |result| < 2.
    a, b, uu = y.cpu().double(), ref.double(), u.double().abs()
    diff = (a - b).abs()
    assert torch.isfinite(a).all()
    if dtype == torch.float32:
        rel = diff.max().item() / b.abs().max().item()
        assert rel <= 1e-5, f"{act} f32: rel {rel:.3e}"
        return
    act_ref = L.ACTIVATIONS[act](g).double()
    bound = (_ulp(b, dtype).double() + _ulp(act_ref, dtype).double() * uu) * 1.0001 + 2e-5 * uu
    over = diff > bound
    assert not over.any(), f"{act} {dtype}: {int(over.sum())} beyond the bound, max {diff.max().item():.3e}"
    small = b.abs() < 2  # where one ulp of the result is below the abs bound
    assert diff[small].max().item() <= 2e-2
    assert (diff > 0).double().mean().item() <= 0.1


def test_layer_errors(cea, dev):
    x = torch.randn(4, 100, device=dev)
    with pytest.raises(ValueError):
        cea.rmsnorm_rope(x, torch.ones(100, device=dev), 1e-5, torch.arange(4, device=dev),
                         torch.ones(4, device=dev), 3)
    with pytest.raises(ValueError):
        cea.silu_mul(x, torch.randn(4, 99, device=dev))
    with pytest.raises(NotImplementedError):
        cea.layers.gated_activation("gelu_new")
    with pytest.raises(NotImplementedError):
        cea.layers.gated_mul(x, x, "swish")
    with pytest.raises(RuntimeError):
        cea.silu_mul(x.cpu(), x.cpu())  # host tensors are refused, never computed on the CPU
