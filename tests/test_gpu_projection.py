"""The fused column-parallel projection GEMM (csrc/gemm.hip) against the oracle
(``F.linear`` on the CPU in the input dtype, tensor_parallel.py:294-295) and against the exact
f64 product.

Bar: every element within the error bound of f32 accumulation rounded once to the dtype,
|y - exact| <= ulp(|exact| + g)/2 + g with g = (K + 2) * 2^-24 * sum_k |x_k w_k| (2^-53 for
f64), and in bf16 / f16 at least 99 % of the elements bit-equal to the oracle (which itself
accumulates in f32; the two differ only where the exact value sits within the accumulation
error of a rounding boundary).  The gated projection must equal the unfused chain
``gated_mul(linear(x, w_gate), linear(x, w_up))`` of this package (same accumulation order,
same activation formulas) bit for bit, except where the last f32 bit of the library's
erf / tanh / exp, inlined into two different kernels, moves ``act(gate)`` across a rounding
boundary of the dtype (at most 0.5 % of the elements, each within 2 ulps); and match the
oracle chain ``act(F.linear(x, w_g)) * F.linear(x, w_u)`` (llama.py:302-305) on at least
98 % of the elements.
"""

import pytest
import torch

from oracle import layers_ref as L

pytestmark = pytest.mark.gpu

ACTS = ["silu", "gelu", "gelu_pytorch_tanh", "relu"]


def _ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23, torch.float64: 52}[dtype]
    tiny = {torch.bfloat16: -133, torch.float16: -24, torch.float32: -149, torch.float64: -1074}[dtype]
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -1000)))
    return torch.pow(2.0, torch.clamp(e - mant, min=tiny))


def _check_linear(got, x, w, b, what, equal_frac=0.99):
    """got [M, N] against the exact product of the (CPU) operands and against the oracle."""
    dtype = got.dtype
    xd, wd = x.double(), w.double()
    exact = xd @ wd.t()
    if b is not None:
        exact = exact + b.double()
    mags = xd.abs() @ wd.abs().t()
    if b is not None:
        mags = mags + b.double().abs()
    k = x.shape[-1]
    eps = 2.0 ** -53 if dtype == torch.float64 else 2.0 ** -24
    g = (k + 2) * eps * mags
    bound = _ulp(exact.abs() + g, dtype) * 0.5 + g
    gd = got.cpu().double()
    err = (gd - exact).abs()
    over = err > bound * 1.0001
    assert not over.any(), f"{what}: {int(over.sum())} elements beyond the bound, max err {err.max().item():.3e}"
    if dtype in (torch.bfloat16, torch.float16) and got.numel():
        ref = L.linear(x, w, b)
        frac = (got.cpu() == ref).double().mean().item()
        assert frac >= equal_frac, f"{what}: only {frac:.4f} of the elements equal the oracle"


def _same_as_chain(y, chain, what):
    diff = y != chain
    if not diff.any():
        return
    assert diff.double().mean().item() <= 0.005, f"{what}: {int(diff.sum())} elements differ"
    yc, cc = y.cpu().double(), chain.cpu().double()
    err = (yc - cc).abs()
    assert bool((err <= 2 * _ulp(cc, y.dtype) * 1.0001).all()), f"{what}: max diff {err.max().item():.3e}"


def _operands(g, m, k, n, dtype, bias=True):
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) / max(k, 1) ** 0.5).to(dtype)
    b = torch.randn(n, generator=g).to(dtype) if bias else None
    return x, w, b


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k,n,bias", [
    (300, 264, 520, True),     # ragged tiles in M and N, a K tail of 8
    (1, 64, 8, False),         # one token
    (513, 1024, 768, True),    # one row past a tile
    (37, 128, 130, True),      # N not a multiple of 4: element stores
    (256, 32, 256, False),     # exactly one tile, one K slice
    (64, 4104, 96, True),      # long K with a tail
])
def test_linear_matches_oracle(cea, dev, dtype, m, k, n, bias):
    g = torch.Generator().manual_seed(m * 7 + k + n)
    x, w, b = _operands(g, m, k, n, dtype, bias)
    y = cea.projection.linear(x.to(dev), w.to(dev), None if b is None else b.to(dev))
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == dtype
    _check_linear(y, x, w, b, f"linear {m}x{k}x{n} {dtype}")


@pytest.mark.parametrize("dtype,m,k,n", [
    (torch.bfloat16, 70, 100, 90),    # K not a multiple of 8: generic kernel
    (torch.float16, 33, 36, 40),
    (torch.float32, 200, 96, 72),
    (torch.float64, 50, 40, 30),
])
def test_linear_generic_kernel(cea, dev, dtype, m, k, n):
    g = torch.Generator().manual_seed(k)
    x, w, b = _operands(g, m, k, n, dtype)
    y = cea.projection.linear(x.to(dev), w.to(dev), b.to(dev))
    torch.cuda.synchronize()
    _check_linear(y, x, w, b, f"generic linear {m}x{k}x{n} {dtype}")


def test_linear_strided_operands_and_preallocated_output(cea, dev):
    """Row-strided x, a column slice of a wider weight (the replicated-token branch's down
    projection reads ``down_proj.weight[:, start:start + count]``, llama.py:315), a
    misaligned x (generic kernel) and a row-strided preallocated output."""
    g = torch.Generator().manual_seed(5)
    dtype = torch.bfloat16
    xb = torch.randn(150, 512 + 64, generator=g).to(dtype)
    wb = (torch.randn(200, 1024, generator=g) / 16).to(dtype)
    b = torch.randn(200, generator=g).to(dtype)
    xd, wd, bd = xb.to(dev), wb.to(dev), b.to(dev)
    for xs, ws in ((xd[:, :512], wd[:, 256:768]), (xd[:, 8:520], wd[:, 0:512]),
                   (xd[:, 1:513], wd[:, 0:512])):
        y = cea.projection.linear(xs, ws, bd)
        torch.cuda.synchronize()
        _check_linear(y, xs.cpu(), ws.cpu(), b, f"strided {xs.stride()} {ws.storage_offset()}")
    out = torch.full((150, 256), 7.0, dtype=dtype, device=dev)
    view = out[:, 16:216]
    cea.projection.linear(xd[:, :512], wd[:, :512], bd, out=view)
    torch.cuda.synchronize()
    _check_linear(view, xb[:, :512], wb[:, :512], b, "preallocated out")
    assert bool((out[:, :16] == 7).all()) and bool((out[:, 216:] == 7).all())


def test_linear_edge_cases(cea, dev):
    dtype = torch.bfloat16
    w = torch.randn(24, 16).to(dtype).to(dev)
    b = torch.randn(24).to(dtype).to(dev)
    y = cea.projection.linear(torch.empty(0, 16, dtype=dtype, device=dev), w, b)
    assert y.shape == (0, 24)
    # no input features: F.linear returns the bias on every row
    y = cea.projection.linear(torch.empty(5, 0, dtype=dtype, device=dev),
                              torch.empty(24, 0, dtype=dtype, device=dev), b)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), b.cpu().expand(5, 24))
    # 3-D input keeps its leading dimensions
    x = torch.randn(2, 3, 16).to(dtype)
    y = cea.projection.linear(x.to(dev), w, b)
    torch.cuda.synchronize()
    assert y.shape == (2, 3, 24)
    _check_linear(y.view(6, 24), x.view(6, 16), w.cpu(), b.cpu(), "3-D input")
    with pytest.raises(ValueError):
        cea.projection.linear(x.to(dev), w[:, :8], b)
    with pytest.raises(ValueError):
        cea.projection.linear(x.to(dev), w, b[:5])


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("dtype,m,k,units,bias", [
    (torch.bfloat16, 300, 264, 200, True),
    (torch.bfloat16, 513, 512, 384, False),
    (torch.float16, 100, 128, 136, True),
    (torch.bfloat16, 40, 100, 50, True),     # generic kernel
    (torch.float32, 40, 64, 48, True),       # generic kernel
])
def test_linear_gated_equals_the_chain(cea, dev, act, dtype, m, k, units, bias):
    g = torch.Generator().manual_seed(units + k)
    x, w, b = _operands(g, m, k, 2 * units, dtype, bias)
    if dtype == torch.float16:
        x = x / 4   # keep gate and up well inside the f16 range
    xd, wd = x.to(dev), w.to(dev)
    bd = None if b is None else b.to(dev)
    layer = cea.FusedColumnParallelLinear(k, [(units, 0, units), (units, 0, units)], None, bias=bias,
                                          dtype=dtype, device=dev)
    with torch.no_grad():
        layer.weight.copy_(wd)
        if bias:
            layer.bias.copy_(bd)
    y = layer.gated(xd, act)
    gate, up = layer(xd)
    chain = cea.layers.gated_mul(gate, up, act)
    torch.cuda.synchronize()
    _same_as_chain(y, chain, f"gated {act} {dtype}")
    # the oracle chain, rounded at the reference's points
    gr = L.linear(x, w[:units], None if b is None else b[:units])
    ur = L.linear(x, w[units:], None if b is None else b[units:])
    ref = L.gated(gr, ur, act)
    if dtype == torch.float32:
        assert torch.allclose(y.cpu(), ref, rtol=1e-4, atol=1e-4)
    else:
        frac = (y.cpu() == ref).double().mean().item()
        assert frac >= 0.98, f"gated {act} {dtype}: only {frac:.4f} equal to the oracle chain"


def test_linear_gated_replicated_token_branch(cea, dev):
    """``units=(start, count)``: gate rows [start, start+count) and up rows
    [I+start, I+start+count) of the fused weight (llama.py:309-314)."""
    g = torch.Generator().manual_seed(11)
    dtype, m, k, units = torch.bfloat16, 96, 256, 320
    x, w, b = _operands(g, m, k, 2 * units, dtype)
    layer = cea.FusedColumnParallelLinear(k, [(units, 0, units), (units, 0, units)], None, bias=True,
                                          dtype=dtype, device=dev)
    with torch.no_grad():
        layer.weight.copy_(w.to(dev))
        layer.bias.copy_(b.to(dev))
    start, count = 64, 136
    y = layer.gated(x.to(dev), "silu", units=(start, count))
    gate = cea.projection.linear(x.to(dev), layer.weight[start:start + count], layer.bias[start:start + count])
    up = cea.projection.linear(x.to(dev), layer.weight[units + start:units + start + count],
                               layer.bias[units + start:units + start + count])
    chain = cea.layers.gated_mul(gate, up, "silu")
    torch.cuda.synchronize()
    assert y.shape == (m, count)
    _same_as_chain(y, chain, "replicated-token branch")


def test_projections_at_the_model_size(cea, dev):
    """The Q/K/V (8192 tokens, 4096 -> 32/8/8 heads x 128) and gate/up (4096 tokens, 4096 ->
    2 x 14336, SiLU) projections of a Llama-3-8B-shaped layer at full size: every output
    element against the exact product's rounding bound and the oracle (Q/K/V), and against
    the oracle's separately rounded projection + activation chain (gate/up), in row blocks of
    1024 tokens."""
    g = torch.Generator().manual_seed(3)
    dtype = torch.bfloat16
    for m, k, n, gated in ((8192, 4096, 6144, False), (4096, 4096, 14336, True)):
        rows = 2 * n if gated else n
        x = torch.randn(m, k, generator=g).to(dtype)
        w = (torch.randn(rows, k, generator=g) / 64).to(dtype)
        b = torch.randn(rows, generator=g).to(dtype) if not gated else None
        xd, wd = x.to(dev), w.to(dev)
        if gated:
            y = cea.projection.linear_gated(xd, wd[:n], wd[n:], act="silu")
        else:
            y = cea.projection.linear(xd, wd, b.to(dev))
        torch.cuda.synchronize()
        yc = y.cpu()
        for r0 in range(0, m, 1024):
            blk = slice(r0, r0 + 1024)
            if gated:
                ref = L.gated(L.linear(x[blk], w[:n]), L.linear(x[blk], w[n:]), "silu")
                frac = (yc[blk] == ref).double().mean().item()
                assert frac >= 0.98, f"gate/up rows {r0}..: {frac:.4f} equal"
            else:
                _check_linear(yc[blk], x[blk], w, b, f"qkv rows {r0}..")


def test_fused_qkv_projection_views_feed_the_kernels(cea, dev):
    """FusedColumnParallelLinear over Q/K/V of a 3-D input: the per-projection outputs are
    column views of one GEMM (strided rows), equal to separate projections, and feed plain
    attention without copies."""
    g = torch.Generator().manual_seed(1)
    B, S, hidden, hq, hkv, d = 2, 70, 512, 8, 2, 64
    layer = cea.FusedColumnParallelLinear(hidden, [(hq * d, 0, hq * d), (hkv * d, 0, hkv * d),
                                                   (hkv * d, 0, hkv * d)], None, bias=True,
                                          dtype=torch.bfloat16, device=dev)
    ws = [(torch.randn(n, hidden, generator=g) / hidden ** 0.5).to(torch.bfloat16)
          for n in (hq * d, hkv * d, hkv * d)]
    bs = [torch.randn(n, generator=g).to(torch.bfloat16) for n in (hq * d, hkv * d, hkv * d)]
    layer.load_full(ws, bs)
    x = torch.randn(B, S, hidden, generator=g).to(torch.bfloat16)
    q, k, v = layer(x.to(dev))
    assert q.shape == (B, S, hq * d) and not k.is_contiguous()
    for got, w, bb in zip((q, k, v), ws, bs):
        _check_linear(got.reshape(B * S, -1), x.view(B * S, hidden), w, bb, "qkv part")
    q4, k4, v4 = q.view(B, S, hq, d), k.view(B, S, hkv, d), v.view(B, S, hkv, d)
    pos = torch.arange(S, device=dev).repeat(B, 1)
    out = cea.attention_fn(q4, k4, v4, pos, pos)
    ref = cea.attention_fn(q4.contiguous(), k4.contiguous(), v4.contiguous(), pos, pos)
    # a decode-shaped call (the last two tokens' queries: the split-KV route) on the views
    dq, dqp = q4[:, -2:], pos[:, -2:]
    dout, dlse = cea.attention_with_lse(dq, k4, v4, dqp, pos)
    dref, dlref = cea.attention_with_lse(dq.contiguous(), k4.contiguous(), v4.contiguous(), dqp, pos)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(dout, dref) and torch.equal(dlse, dlref)
