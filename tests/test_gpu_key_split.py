"""Key-split prefill launches, through the C ABI and the operator library.

Short query blocks against long key blocks (a prefill chunk against the cache before it, or a
few tokens with more query rows than the split-KV decode kernels take) give too few
query blocks to fill the device; the prefill route then deals the key tiles to several groups
of workgroups and merges their partial (out, lse) pairs.  Each case is checked against the
oracle at the bf16 tolerances, against the unsplit launch (the same call given only the
tile-summary workspace, so it cannot split), and through the operator library and plain
attention (bf16 out).
"""

from ctypes import byref

import pytest
import torch

from _cases import assert_attention_close
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

CASES = [
    # B, Sq, Sk, Hq, Hkv, D, positions, causal
    (1, 128, 20000, 32, 8, 128, "chunk", True),   # a 128-token prefill chunk at batch 1
    (2, 40, 3000, 8, 1, 64, "chunk", True),       # 8 query heads per KV head: 320 rows
    (1, 20, 9000, 8, 8, 128, "chunk", True),      # 20 tokens, one query head per KV head
    (1, 100, 7000, 16, 4, 128, "padded", True),   # padded keys and padded query rows
    (1, 64, 5000, 8, 2, 64, "chunk", False),      # no causal rule
]


def _tile_ws(B, Sk):
    """Bytes of the per-tile key-position summaries alone (32 bytes per 64-key tile and batch
    row, rounded up to 256)."""
    return -(-B * -(-Sk // 64) * 32 // 256) * 256


def _inputs(B, Sq, Sk, Hq, Hkv, D, kind):
    g = torch.Generator().manual_seed(Sk + Sq)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16)
    kp = torch.arange(Sk).repeat(B, 1)
    if kind == "padded":
        kp[:, Sk - 1500:] = -1
        qp = torch.arange(Sk - 1500 - Sq, Sk - 1500).repeat(B, 1)
        qp[:, -10:] = -1
    else:
        qp = torch.arange(Sk - Sq, Sk).repeat(B, 1)
    return q, k, v, qp, kp


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}-Sq{}-Sk{}-H{}/{}-D{}-{}-{}".format(
    *c[:7], "c" if c[7] else "nc"))
def test_key_split_matches_oracle_and_unsplit(cea, dev, case):
    B, Sq, Sk, Hq, Hkv, D, kind, causal = case
    q, k, v, qp, kp = _inputs(B, Sq, Sk, Hq, Hkv, D, kind)
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp, causal=causal)
    nat = cea._native
    lib = nat.load_library()
    t = [x.to(dev) for x in (q, k, v, qp, kp)]
    args = [nat.tensor_arg(x) for x in t]
    stream = nat.stream_of(dev)
    full = lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, 1)
    assert full > _tile_ws(B, Sk)  # the plan splits the keys
    res = []
    for ws_bytes in (full, _tile_ws(B, Sk)):
        print(f"key-split test: case={case} workspace={ws_bytes}", flush=True)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        out = torch.full((B, Sq, Hq, D), float("nan"), device=dev)
        lse = torch.full((B, Hq, Sq), float("nan"), device=dev)
        o, l = nat.tensor_arg(out), nat.tensor_arg(lse)
        rc = lib.cea_attention_with_lse(*(byref(a) for a in args), int(causal), D ** -0.5, None, 0,
                                        byref(o), byref(l), 0, ws.data_ptr(), ws.numel(), stream)
        assert rc == 0, nat.last_error()
        res.append((out, lse))
    torch.cuda.synchronize()
    (so, sl), (uo, ul) = res
    assert_attention_close(so, sl, ro, rl, torch.bfloat16, f"{case} split")
    assert_attention_close(uo, ul, ro, rl, torch.bfloat16, f"{case} unsplit")
    fin = torch.isfinite(ul)
    assert torch.equal(torch.isfinite(sl), fin)
    # the value products take the probabilities in bf16, rounded against each split's own
    # running maximum: outputs agree to that rounding (2^-8 relative), lse sums are f32
    assert (so - uo).abs().max().item() <= 4e-3
    assert (sl[fin] - ul[fin]).abs().max().item() <= 1e-5
    # the operator library takes the same route; plain attention rounds the merged output
    po, pl = cea.attention_with_lse(*t, causal=causal)
    plain = cea.attention.attention(*t, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(po, so) and torch.equal(pl, sl)
    assert plain.dtype == torch.bfloat16 and torch.equal(plain, so.to(torch.bfloat16))
