"""The column views of the fused Q/K/V projection output (tensor_parallel.py:294-295) feed the
attention kernels without copies: attention on the strided views equals attention on
contiguous copies, bit for bit.  (The GEMM itself is PyTorch's and is not tested here.)
"""

import pytest
import torch

from oracle import layers_ref as L

pytestmark = pytest.mark.gpu


def _ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[dtype]
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -24)))
    return torch.pow(2.0, e - mant)


def _check(got: torch.Tensor, want: torch.Tensor):
    dtype = got.dtype
    got, want = got.cpu().double(), want.double()
    if dtype == torch.float32:
        assert (got - want).abs().max().item() <= 1e-5 * want.abs().max().item()
        return
    err = (got - want).abs()
    assert bool((err <= _ulp(want, dtype) + 1e-4 * want.abs().max()).all()), err.max().item()


def test_fused_qkv_projection_views_feed_the_kernels(cea, dev):
    """FusedColumnParallelLinear over Q/K/V of a 3-D input: the per-projection outputs are
    column views of one GEMM (strided rows), equal to separate projections, and feed the
    KV-cache append (rotary of K) and plain attention without copies."""
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
        _check(got, L.linear(x.float(), w.float(), bb.float()).to(torch.bfloat16))
    # the views go into the kernels as they are
    q4, k4, v4 = q.view(B, S, hq, d), k.view(B, S, hkv, d), v.view(B, S, hkv, d)
    pos = torch.arange(S, device=dev).repeat(B, 1)
    out = cea.attention_fn(q4, k4, v4, pos, pos)
    ref = cea.attention_fn(q4.contiguous(), k4.contiguous(), v4.contiguous(), pos, pos)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
