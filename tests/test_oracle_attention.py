"""Pins of the attention oracle (oracle/attention_ref.py) on the CPU.

Each oracle function is checked against something that does not share its code:
* the fp64 brute force of tests/_brute.py (definition of masked softmax attention, one key
  at a time) on every mask pattern, GQA/MQA/irregular head maps, scales and kv_block splits,
  through both of the reference's routes (CPU flash op and materialised scores);
* torch's scaled_dot_product_attention, the reference's own known answer
  (tests/test_attention.py:19-25 of the reference);
* the exact invariants of the reference's tests: repeat-interleaved K/V == kv_map
  (test_attention.py:28-34), merge of disjoint key subsets == unsplit attention (:37-49),
  empty rows are (0, -inf) and merging with an empty partial is the identity (:52-63),
  default scale 1/sqrt(D) (:66-69);
* planted mistakes: each test at the end swaps one oracle function for a wrong copy
  (off-by-one causal rule, padding ignored, transposed head map, swapped merge weights,
  max in place of logsumexp, empty-row fix-up dropped, scale dropped) and shows the pins
  above reject it.
All fp64 checks use 1e-12 (the reference's tolerance); f32 uses normwise rel 1e-5.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import _brute
from _cases import Case
from oracle import attention_ref as ref

F64 = torch.float64

PIN_CASES = [
    Case(2, 9, 9, 4, 2, 8, "aligned"),
    Case(2, 9, 9, 4, 2, 8, "left_pad"),
    Case(2, 10, 10, 6, 3, 4, "right_pad"),
    Case(2, 8, 6, 4, 4, 8, "zigzag"),
    Case(3, 1, 17, 8, 2, 8, "decode"),
    Case(2, 7, 11, 4, 2, 4, "random", causal=True, seed=3),
    Case(2, 7, 11, 4, 2, 4, "random", causal=False, seed=4),
    Case(1, 5, 5, 2, 1, 4, "all_pad"),
    Case(2, 9, 9, 6, 1, 4, "left_pad", seed=5),                        # MQA
    Case(1, 6, 6, 6, 2, 4, "random", kv_map=(0, 1, 1, 1, 1, 1), seed=6),  # irregular map
    Case(2, 6, 6, 4, 2, 8, "random", scale=0.3, seed=7),
]


def _errors(out, lse, bo, bl):
    """(max |out - bo|, max |lse - bl| over finite entries); inf if the -inf patterns differ."""
    out, lse = out.double().numpy(), lse.double().numpy()
    if not np.array_equal(np.isfinite(lse), np.isfinite(bl)):
        return math.inf, math.inf
    fin = np.isfinite(bl)
    dl = float(np.abs(lse[fin] - bl[fin]).max()) if fin.any() else 0.0
    do = float(np.abs(out - bo).max()) if out.size else 0.0
    return do, dl


def _oracle_vs_brute(case: Case, route: str, kv_block=None, dtype=F64):
    q, k, v, qp, kp = case.tensors(dtype)
    out, lse = ref.attention_with_lse(q, k, v, qp, kp, causal=case.causal, scale=case.scale,
                                      kv_map=case.kv_map, kv_block=kv_block, route=route)
    bo, bl = _brute.attention(q.double(), k.double(), v.double(), qp, kp, case.causal,
                              case.scale, case.kv_map)
    return _errors(out, lse, bo, bl), (bo, bl)


@pytest.mark.parametrize("route", ["flash", "math"])
@pytest.mark.parametrize("case", PIN_CASES, ids=str)
def test_oracle_matches_brute_force_f64(case, route):
    (do, dl), _ = _oracle_vs_brute(case, route)
    assert do <= 1e-12 and dl <= 1e-12, (do, dl)


@pytest.mark.parametrize("case", PIN_CASES[:7], ids=str)
def test_oracle_kv_block_matches_brute_force(case):
    (do, dl), _ = _oracle_vs_brute(case, "flash", kv_block=3)
    assert do <= 1e-12 and dl <= 1e-12, (do, dl)


@pytest.mark.parametrize("case", PIN_CASES[:7], ids=str)
def test_oracle_f32_matches_brute_force(case):
    (do, dl), (bo, bl) = _oracle_vs_brute(case, "flash", dtype=torch.float32)
    fin = np.isfinite(bl)
    assert do / max(np.abs(bo).max(), 1e-30) <= 1e-5
    if fin.any():
        assert dl / np.abs(bl[fin]).max() <= 1e-5


@pytest.mark.parametrize("scale", [-0.5, 0.0])
def test_oracle_nonpositive_scale_on_the_scores_route(scale):
    """The scores route handles any scale; the CPU flash op returns NaN when is_causal=True
    and scale <= 0 (a torch property, shown here), so those cases use the scores route."""
    case = Case(2, 6, 6, 4, 2, 8, "random", scale=scale, seed=8)
    (do, dl), _ = _oracle_vs_brute(case, "math")
    assert do <= 1e-12 and dl <= 1e-12
    q = torch.randn(1, 2, 3, 4, dtype=F64)
    o, l = ref._FLASH_CPU(q, q, q, 0.0, True, attn_mask=None, scale=scale)
    assert torch.isnan(o).any() or torch.isnan(l).any()


def test_empty_inputs():
    q = torch.randn(2, 3, 4, 8, dtype=F64)
    k = torch.randn(2, 0, 2, 8, dtype=F64)
    out, lse = ref.attention_with_lse(q, k, k, torch.zeros(2, 3, dtype=torch.long),
                                      torch.zeros(2, 0, dtype=torch.long))
    assert out.shape == (2, 3, 4, 8) and torch.all(out == 0)
    assert lse.shape == (2, 4, 3) and torch.all(lse == float("-inf"))
    out, lse = ref.attention_with_lse(q[:, :0], torch.randn(2, 5, 2, 8, dtype=F64),
                                      torch.randn(2, 5, 2, 8, dtype=F64),
                                      torch.zeros(2, 0, dtype=torch.long), torch.arange(5).repeat(2, 1))
    assert out.shape == (2, 0, 4, 8) and lse.shape == (2, 4, 0)


def _rand(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=F64)


@pytest.mark.parametrize("causal", [True, False])
def test_plain_attention_matches_sdpa(causal):
    """Known answer of the reference (test_attention.py:19-25)."""
    q, k, v = _rand(2, 7, 4, 8, seed=1), _rand(2, 7, 4, 8, seed=2), _rand(2, 7, 4, 8, seed=3)
    pos = torch.arange(7).repeat(2, 1)
    ours = ref.plain_attention(q, k, v, pos, pos, causal=causal)
    want = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                          is_causal=causal).transpose(1, 2)
    torch.testing.assert_close(ours, want)
    out, _ = ref.attention_with_lse(q, k, v, pos, pos, causal=causal)
    torch.testing.assert_close(out, want)


def test_gqa_map_equals_repeated_kv():
    """test_attention.py:28-34."""
    q, k, v = _rand(1, 9, 6, 4, seed=4), _rand(1, 9, 2, 4, seed=5), _rand(1, 9, 2, 4, seed=6)
    pos = torch.arange(9).view(1, 9)
    want = ref.plain_attention(q, k.repeat_interleave(3, 2), v.repeat_interleave(3, 2), pos, pos)
    torch.testing.assert_close(ref.plain_attention(q, k, v, pos, pos), want)
    torch.testing.assert_close(ref.plain_attention(q, k, v, pos, pos, kv_map=[0, 0, 0, 1, 1, 1]), want)
    torch.testing.assert_close(ref.plain_attention(q, k, v, pos, pos, kv_block=2), want)


def test_merge_of_disjoint_key_sets_is_exact():
    """test_attention.py:37-49."""
    q, k, v = _rand(2, 5, 3, 4, seed=7), _rand(2, 12, 3, 4, seed=8), _rand(2, 12, 3, 4, seed=9)
    qpos = torch.arange(7, 12).repeat(2, 1)
    kpos = torch.arange(12).repeat(2, 1)
    full, full_lse = ref.attention_with_lse(q, k, v, qpos, kpos)
    idx = torch.randperm(12, generator=torch.Generator().manual_seed(0))
    parts = [idx[:3], idx[3:8], idx[8:]]
    outs, lses = zip(*[ref.attention_with_lse(q, k[:, p], v[:, p], qpos, kpos[:, p]) for p in parts])
    out, lse = ref.merge_many(list(outs), list(lses))
    torch.testing.assert_close(out, full, atol=1e-12, rtol=0)
    torch.testing.assert_close(lse, full_lse, atol=1e-12, rtol=0)
    out2, _ = ref.merge_pair(*ref.merge_pair(outs[0], lses[0], outs[1], lses[1]), outs[2], lses[2])
    torch.testing.assert_close(out2, full, atol=1e-12, rtol=0)


def test_padding_rows_and_empty_partial():
    """test_attention.py:52-63."""
    q, k, v = _rand(1, 4, 2, 4, seed=10), _rand(1, 4, 2, 4, seed=11), _rand(1, 4, 2, 4, seed=12)
    pos = torch.tensor([[-1, -1, 0, 1]])
    out, lse = ref.attention_with_lse(q, k, v, pos, pos)
    assert torch.isfinite(out).all()
    assert torch.all(out[:, :2] == 0) and torch.isinf(lse[..., :2]).all()
    want = ref.plain_attention(q[:, 2:], k[:, 2:], v[:, 2:], pos[:, 2:], pos[:, 2:])
    torch.testing.assert_close(out[:, 2:], want)
    eo, el = ref.attention_with_lse(q, k[:, :0], v[:, :0], pos, pos[:, :0])
    merged, mlse = ref.merge_pair(out, lse, eo, el)
    torch.testing.assert_close(merged, out)
    merged, mlse = ref.merge_many([eo, out, eo], [el, lse, el])
    torch.testing.assert_close(merged, out)
    assert torch.equal(torch.isinf(mlse), torch.isinf(lse))


def test_scale_default():
    """test_attention.py:66-69."""
    q, k, v = _rand(1, 3, 1, 16, seed=13), _rand(1, 3, 1, 16, seed=14), _rand(1, 3, 1, 16, seed=15)
    pos = torch.arange(3).view(1, 3)
    torch.testing.assert_close(ref.plain_attention(q, k, v, pos, pos),
                               ref.plain_attention(q, k, v, pos, pos, scale=0.25))


def test_dispatch_modes_and_chunks():
    """attention.py:116-141 on the measured workloads' position patterns."""
    a = torch.arange(512).view(1, 512)
    assert ref.dispatch_mode(a, a, True) == "causal"             # aligned prefill
    assert ref.dispatch_mode(a, a, False) == "none"
    zig_q = torch.cat([torch.arange(4096), torch.arange(28672, 32768)]).view(1, -1)
    assert ref.dispatch_mode(zig_q, zig_q, True) == "mask"        # zigzag share
    cache = torch.where(torch.arange(100) < 60, torch.arange(100), -1).view(1, 100)
    assert ref.dispatch_mode(torch.tensor([[59]]), cache, True) == "mask"   # decode cache
    # right-padded 65536-token share: chunks of 4Mi // 65536 = 64 query rows -> 1024 chunks
    pos = torch.where(torch.arange(65536) < 40000, torch.arange(65536), -1).view(1, -1)
    chunks = [(lo, hi) for lo, hi, _, _ in ref.query_chunks(pos[:, :4096], pos, True)]
    assert chunks[0] == (0, 64) and len(chunks) == 4096 // 64
    assert ref.MASK_CHUNK_ELEMENTS // 65536 == 64


def test_nothing_visible_rule():
    """attention.py:104-113: skip iff no valid key or max q_pos < min valid k_pos (causal)."""
    qp = torch.tensor([[3, 4]])
    assert ref.nothing_visible(qp, torch.tensor([[-1, -1]]))
    assert ref.nothing_visible(qp, torch.tensor([[5, 9]]))
    assert not ref.nothing_visible(qp, torch.tensor([[5, 9]]), causal=False)
    assert not ref.nothing_visible(qp, torch.tensor([[4, 9]]))
    assert ref.nothing_visible(qp, torch.zeros(1, 0, dtype=torch.long))


# ---- planted mistakes: each must be rejected by the pins above ---------------------------

def _suite_error(route="flash", cases=PIN_CASES):
    worst = 0.0
    for case in cases:
        (do, dl), _ = _oracle_vs_brute(case, route)
        worst = max(worst, do, dl)
    return worst


def test_planted_off_by_one_causal_rule_is_caught(monkeypatch):
    def strict(q_pos, k_pos, causal=True):
        ok = (k_pos >= 0)[:, None, None, :]
        if causal:
            ok = ok & (k_pos[:, None, None, :] < q_pos[:, None, :, None])
        return ok.expand(q_pos.shape[0], 1, q_pos.shape[1], k_pos.shape[1])

    assert _suite_error() <= 1e-12
    monkeypatch.setattr(ref, "visible", strict)
    assert _suite_error() > 1e-3
    assert _suite_error("math") > 1e-3


def test_planted_padding_ignored_is_caught(monkeypatch):
    def no_pad(q_pos, k_pos, causal=True):
        ok = torch.ones(k_pos.shape, dtype=torch.bool)[:, None, None, :]
        if causal:
            ok = ok & (k_pos[:, None, None, :] <= q_pos[:, None, :, None])
        return ok.expand(q_pos.shape[0], 1, q_pos.shape[1], k_pos.shape[1])

    monkeypatch.setattr(ref, "visible", no_pad)
    assert _suite_error("math") > 1e-3


def test_planted_transposed_head_map_is_caught(monkeypatch):
    def modulo_map(x, hq, kv_map=None):
        return x.index_select(2, torch.tensor([h % x.shape[2] for h in range(hq)]))

    monkeypatch.setattr(ref, "group_of", lambda hq, hkv, kv_map=None: None)
    monkeypatch.setattr(ref, "expand_heads", modulo_map)
    assert _suite_error() > 1e-3


def test_planted_swapped_merge_weights_are_caught(monkeypatch):
    good = ref.merge_pair

    def swapped(out_a, lse_a, out_b, lse_b):
        return good(out_a, lse_b, out_b, lse_a)

    monkeypatch.setattr(ref, "merge_pair", swapped)
    errs = [_oracle_vs_brute(c, "flash", kv_block=3)[0] for c in PIN_CASES[:7]]
    assert max(max(e) for e in errs) > 1e-3


def test_planted_max_for_logsumexp_is_caught(monkeypatch):
    def max_merge(outs, lses):
        st = torch.stack(list(lses))
        lse = st.amax(dim=0)
        safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
        w = torch.exp(st - safe)
        return sum(o * wi.transpose(1, 2).unsqueeze(-1) for o, wi in zip(outs, w)), lse

    monkeypatch.setattr(ref, "merge_many", max_merge)
    with pytest.raises(AssertionError):
        test_merge_of_disjoint_key_sets_is_exact()


def test_planted_missing_empty_row_fixup_is_caught(monkeypatch):
    monkeypatch.setattr(ref, "empty_rows_fixup", lambda o, l, mask: (o, l))
    assert _suite_error() > 1e-3


def test_planted_dropped_scale_is_caught(monkeypatch):
    class NoSqrt:
        @staticmethod
        def sqrt(x):
            return 1.0

    monkeypatch.setattr(ref, "math", NoSqrt)
    assert _suite_error(cases=PIN_CASES[:3]) > 1e-3
