"""The no-allocation entry point cea_attention_with_lse_noalloc, through the C ABI.

It must return exactly what cea_attention_with_lse returns (same kernels; only the scratch
differs: a static per-GPU device array instead of the caller's workspace).  Checked bit for
bit on two calls in a row, the second with a smaller input, for both scratch users: the
prefill route (per-tile key-position summaries) and the split-KV decode route (chunk
partials, visibility words, tile masks), plus the in-place accumulate form; a call whose
scratch need exceeds the array is refused before anything is launched.
"""

from __future__ import annotations

import ctypes
from ctypes import byref

import pytest
import torch

pytestmark = pytest.mark.gpu

ENOSPACE = -4
SCRATCH_BYTES = 32 << 20


def _inputs(B, Sq, Sk, Hq, Hkv, D, seed, decode):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16)
    if decode:  # one new token per sequence against a -1-tailed cache
        lens = torch.randint(1, Sk + 1, (B,), generator=g)
        slots = torch.arange(Sk).view(1, Sk)
        kp = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
        qp = (lens - 1).view(-1, 1)
    else:  # causal prefill with right padding
        kp = torch.arange(Sk).repeat(B, 1)
        kp[:, Sk - Sk // 7:] = -1
        qp = torch.arange(Sk - Sq, Sk).repeat(B, 1)
    return q, k, v, qp, kp


def _run(cea, fn_name, tensors, out, lse, accumulate=0):
    nat = cea._native
    lib = nat.load_library()
    q, k, v, qp, kp = tensors
    args = [nat.tensor_arg(t) for t in (q, k, v, qp, kp)]
    o, l = nat.tensor_arg(out), nat.tensor_arg(lse)
    stream = nat.stream_of(q.device)
    scale = 1.0 / q.shape[-1] ** 0.5
    if fn_name == "cea_attention_with_lse":
        B, Sq, Hq, D = q.shape
        ws_bytes = lib.cea_attention_workspace_bytes(B, Sq, Hq, k.shape[1], k.shape[2], D, 1)
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=q.device)
        rc = lib.cea_attention_with_lse(*(byref(a) for a in args), 1, scale, None, 0, byref(o),
                                        byref(l), accumulate, ws.data_ptr(), ws.numel(), stream)
    else:
        rc = lib.cea_attention_with_lse_noalloc(*(byref(a) for a in args), 1, scale, None, 0,
                                                byref(o), byref(l), accumulate, stream)
    return rc


def _check_same(cea, dev, shape, seed, decode):
    B, Sq, Sk, Hq, Hkv, D = shape
    t = tuple(x.to(dev) for x in _inputs(B, Sq, Sk, Hq, Hkv, D, seed, decode))
    lib = cea._native.load_library()
    need = lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, 1)
    assert need <= SCRATCH_BYTES, need
    outs = []
    for fn in ("cea_attention_with_lse", "cea_attention_with_lse_noalloc"):
        out = torch.full((B, Sq, Hq, D), float("nan"), device=dev)
        lse = torch.full((B, Hq, Sq), float("nan"), device=dev)
        print(f"no-alloc test: {fn} shape={shape} decode={decode}", flush=True)
        rc = _run(cea, fn, t, out, lse)
        assert rc == 0, (fn, rc, cea._native.last_error())
        # the accumulate form merges a second, shifted-key call into the running pair
        t2 = (t[0], t[1].flip(1), t[2].flip(1), t[3], t[4])
        rc = _run(cea, fn, t2, out, lse, accumulate=1)
        assert rc == 0, (fn, rc, cea._native.last_error())
        torch.cuda.synchronize()
        outs.append((out.cpu(), lse.cpu()))
    (o1, l1), (o2, l2) = outs
    assert torch.isfinite(o1).all()
    assert torch.equal(o1, o2) and torch.equal(l1, l2), shape


@pytest.mark.parametrize("decode", [False, True], ids=["prefill-route", "decode-route"])
def test_noalloc_matches_workspace_entry(cea, dev, decode):
    if decode:  # split-KV decode: B sequences, one query each, GQA 32/8
        first, second = (8, 1, 30000, 32, 8, 128), (3, 1, 4000, 32, 8, 128)
    else:      # MFMA prefill with tile summaries
        first, second = (2, 700, 3000, 8, 2, 128), (1, 129, 500, 8, 2, 128)
    _check_same(cea, dev, first, seed=1, decode=decode)
    _check_same(cea, dev, second, seed=2, decode=decode)


def test_noalloc_refuses_oversized_calls(cea, dev):
    """64 sequences of a 32768-slot cache need more chunk partials than the static scratch
    holds: refused with CEA_ENOSPACE before any launch (broadcast views, nothing allocated
    at full size, nothing written)."""
    lib = cea._native.load_library()
    B, Sk, Hq, Hkv, D = 64, 32768, 32, 8, 128
    need = lib.cea_attention_workspace_bytes(B, 1, Hq, Sk, Hkv, D, 1)
    assert need > SCRATCH_BYTES
    q = torch.zeros(1, 1, Hq, D, dtype=torch.bfloat16, device=dev).expand(B, 1, Hq, D)
    k = torch.zeros(1, Sk, Hkv, D, dtype=torch.bfloat16, device=dev).expand(B, Sk, Hkv, D)
    qp = torch.zeros(1, 1, dtype=torch.int64, device=dev).expand(B, 1)
    kp = torch.zeros(1, Sk, dtype=torch.int64, device=dev).expand(B, Sk)
    out = torch.zeros(B, 1, Hq, D, device=dev)
    lse = torch.zeros(B, Hq, 1, device=dev)
    rc = _run(cea, "cea_attention_with_lse_noalloc", (q, k, k, qp, kp), out, lse)
    assert rc == ENOSPACE
    assert "static scratch" in cea._native.last_error()
    torch.cuda.synchronize()
    assert bool((out == 0).all()) and bool((lse == 0).all())


def test_noalloc_takes_f32_decode_shapes(cea, dev):
    """A float32 call of a decode shape needs no split-KV partials (that route is bf16 / f16
    only): the no-allocation entry runs it and matches the workspace entry exactly, twice in
    a row, the second call smaller."""
    nat = cea._native
    lib = nat.load_library()
    for shape in ((4, 1, 9000, 32, 8, 128), (2, 1, 3000, 32, 8, 128)):
        B, Sq, Sk, Hq, Hkv, D = shape
        t = tuple(x.to(dev) for x in _inputs(B, Sq, Sk, Hq, Hkv, D, seed=B, decode=True))
        t = (t[0].float(), t[1].float(), t[2].float(), t[3], t[4])
        assert lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, 0) <= SCRATCH_BYTES
        res = []
        for fn in ("cea_attention_with_lse", "cea_attention_with_lse_noalloc"):
            out = torch.full((B, Sq, Hq, D), float("nan"), device=dev)
            lse = torch.full((B, Hq, Sq), float("nan"), device=dev)
            args = [nat.tensor_arg(x) for x in t]
            o, l = nat.tensor_arg(out), nat.tensor_arg(lse)
            stream = nat.stream_of(dev)
            print(f"no-alloc test: {fn} f32 shape={shape}", flush=True)
            if fn == "cea_attention_with_lse":
                need = lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, 0)
                ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
                rc = lib.cea_attention_with_lse(*(byref(a) for a in args), 1, D ** -0.5, None, 0,
                                                byref(o), byref(l), 0, ws.data_ptr(), ws.numel(), stream)
            else:
                rc = lib.cea_attention_with_lse_noalloc(*(byref(a) for a in args), 1, D ** -0.5, None,
                                                        0, byref(o), byref(l), 0, stream)
            assert rc == 0, (fn, rc, nat.last_error())
            torch.cuda.synchronize()
            res.append((out.cpu(), lse.cpu()))
        assert torch.isfinite(res[0][0]).all()
        assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])

