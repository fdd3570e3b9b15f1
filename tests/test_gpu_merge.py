"""GPU parity of the exact LSE merges (merge_attention, merge_attention_list) against the
oracle's merges (attention.py:242-264), on partials with empty (-inf) rows, strided views
and more partials than one kernel launch takes.  f64: max abs <= 1e-12; f32: normwise
rel <= 1e-5 (tests/_cases.py); empty rows exactly (0, -inf)."""

from __future__ import annotations

import pytest
import torch

from _cases import assert_attention_close
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _partials(n, dtype, B=2, Sq=5, H=3, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    outs, lses = [], []
    for i in range(n):
        o = torch.randn(B, Sq, H, D, generator=g, dtype=torch.float64)
        l = 3 * torch.randn(B, H, Sq, generator=g, dtype=torch.float64)
        empty = torch.rand(B, H, Sq, generator=g) < 0.3
        empty[0, 0, 0] = True          # one row empty in every partial
        l = l.masked_fill(empty, float("-inf"))
        o = o.masked_fill(empty.transpose(1, 2).unsqueeze(-1), 0.0)
        outs.append(o.to(dtype))
        lses.append(l.to(dtype))
    return outs, lses


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32], ids=["float64", "float32"])
@pytest.mark.parametrize("n", [2, 3, 7, 16, 17, 40])
def test_merge_list_matches_oracle(cea, dev, n, dtype):
    outs, lses = _partials(n, dtype, seed=n)
    out, lse = cea.merge_attention_list([o.to(dev) for o in outs], [l.to(dev) for l in lses])
    ro, rl = ref.merge_many(outs, lses)
    torch.cuda.synchronize()
    assert out.dtype == dtype and lse.dtype == dtype
    assert_attention_close(out, lse, ro, rl, dtype, f"merge of {n}")
    assert out[0, 0, 0].abs().max().item() == 0 and lse[0, 0, 0].item() == float("-inf")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32], ids=["float64", "float32"])
def test_pairwise_merge_matches_oracle_on_views(cea, dev, dtype):
    outs, lses = _partials(2, dtype, D=128, seed=5)
    big = torch.zeros(2, 5, 6, 128, dtype=dtype)
    big[:, :, 1:4] = outs[0]
    oa = big.to(dev)[:, :, 1:4]                      # strided along heads
    la = lses[0].transpose(1, 2).contiguous().to(dev).transpose(1, 2)  # [B, H, Sq] view
    assert not oa.is_contiguous() and not la.is_contiguous()
    out, lse = cea.merge_attention(oa, la, outs[1].to(dev), lses[1].to(dev))
    ro, rl = ref.merge_pair(outs[0], lses[0], outs[1], lses[1])
    torch.cuda.synchronize()
    assert_attention_close(out, lse, ro, rl, dtype, "pairwise")


def test_merge_is_pure_and_validates(cea, dev):
    outs, lses = _partials(3, torch.float32, seed=9)
    od = [o.to(dev) for o in outs]
    ld = [l.to(dev) for l in lses]
    before = [o.clone() for o in od]
    cea.merge_attention_list(od, ld)
    cea.merge_attention(od[0], ld[0], od[1], ld[1])
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(od, before))
    one = cea.merge_attention_list(od[:1], ld[:1])
    assert one[0] is od[0] and one[1] is ld[0]
    with pytest.raises(ValueError):
        cea.merge_attention_list([], [])
    with pytest.raises(ValueError):
        cea.merge_attention_list(od, ld[:2])
    with pytest.raises(ValueError):
        cea.merge_attention(od[0], ld[0], od[1][:, :2], ld[1][:, :, :2])
