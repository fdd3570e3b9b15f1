"""GPU parity of the wire-format kernels, through the C ABI:

* ``cea_ulysses_scatter`` / ``cea_ulysses_gather`` (sequence_parallel.py:163-194) against the
  oracle's restatement of the send lists, all-to-all and concatenations: bit-exact copies for
  every dtype, uneven sequence and head splits, batch 2, strided shard views, wire rounding;
  and at the Ulysses workload's full size (65536 tokens, sp=8) against slicing;
* ``cea_pack_partial`` / ``cea_merge_packed`` (sequence_parallel.py:275-280): the packed
  message is exact, the in-place merge equals ``merge_attention_list`` of the unpacked
  views bit for bit and the oracle within the f32 tolerance, and the distributed-KV decode
  workload through the packed route equals the fused route.
"""

import pytest
import torch

from oracle import attention_ref as ref
from oracle import sp_ref

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32, torch.float64]


def _group(cea, shards, rank, wire_dtype=None):
    grp = cea.LocalGroup(len(shards), rank, wire_dtype=wire_dtype)
    for j, (q, k, v, p) in enumerate(shards):
        grp.set_shard(j, q=q, k=k, v=v, pos=p)
    return grp


def _make(cea, dtype, B, S, hq, hkv, D, world, weights, kind, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, hq, D, generator=g, dtype=torch.float64).to(dtype)
    k = torch.randn(B, S, hkv, D, generator=g, dtype=torch.float64).to(dtype)
    v = torch.randn(B, S, hkv, D, generator=g, dtype=torch.float64).to(dtype)
    pos = torch.arange(S).repeat(B, 1)
    pos[-1, -3:] = -1
    layout = cea.SequenceLayout(S, world, weights, kind)
    shards = [tuple(layout.shard(t, r) for t in (q, k, v, pos)) for r in range(world)]
    return layout, shards


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("world,weights,kind,hq,hkv,D",
                         [(2, None, "contiguous", 8, 4, 128), (3, [3, 2, 1], "zigzag", 6, 3, 64),
                          (4, [1, 1, 2, 3], "contiguous", 12, 4, 20), (8, None, "zigzag", 64, 16, 128)])
def test_ulysses_scatter_gather_match_oracle(cea, dev, dtype, world, weights, kind, hq, hkv, D):
    B, S = 2, 8 * 37
    layout, shards = _make(cea, dtype, B, S, hq, hkv, D, world, weights, kind)
    heads = cea.partition_heads(hq, hkv, weights or world)
    shards_d = [tuple(t.to(dev) for t in sh) for sh in shards]
    outs, outs_ref = [], []
    for r in range(world):
        got = cea.ulysses_scatter(*shards_d[r], _group(cea, shards_d, r), layout.sizes, heads)
        want = sp_ref.ulysses_scatter(shards, heads, r)
        torch.cuda.synchronize()
        for a, b_ in zip(got, want):
            assert a.dtype == b_.dtype and torch.equal(a.cpu(), b_), f"scatter rank {r}"
        outs.append(got[0] * 2)  # any per-rank head output: the scattered queries, doubled
        outs_ref.append(want[0] * 2)
    for r in range(world):
        grp = _group(cea, shards_d, r)
        for j in range(world):  # what the other ranks send back in the second all-to-all
            grp.set_shard(j, out_heads=outs[j])
        got = cea.ulysses_gather(outs[r], grp, layout.sizes, heads)
        want = sp_ref.ulysses_gather(outs_ref, layout.sizes, r)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want), f"gather rank {r}"


def test_ulysses_scatter_strided_views_and_wire_rounding(cea, dev):
    """Shards that are head slices of a fused QKV output (token stride > heads * D, non-16-byte
    multiples), and bf16 wire compression of every piece (comm.py:468-486)."""
    world, hq, hkv, D, B, S = 3, 6, 3, 40, 2, 61
    g = torch.Generator().manual_seed(3)
    fused = torch.randn(B, S, hq + 2 * hkv + 1, D, generator=g, dtype=torch.float32)
    q, k, v = fused[:, :, :hq], fused[:, :, hq:hq + hkv], fused[:, :, hq + hkv:hq + 2 * hkv]
    pos = torch.arange(S).repeat(B, 1)
    layout = cea.SequenceLayout(S, world, [2, 1, 1], "contiguous")
    heads = cea.partition_heads(hq, hkv, [2, 1, 1])
    shards = [tuple(layout.shard(t, r) for t in (q, k, v, pos)) for r in range(world)]
    shards_d = [tuple(t.to(dev) for t in sh) for sh in shards]
    fd = fused.to(dev)
    # device shards as views of the device fused tensor
    qd, kd, vd = fd[:, :, :hq], fd[:, :, hq:hq + hkv], fd[:, :, hq + hkv:hq + 2 * hkv]
    shards_v = [tuple(layout.shard(t, r) for t in (qd, kd, vd, pos.to(dev))) for r in range(world)]
    assert not shards_v[0][0].is_contiguous()
    rounded = [tuple(t.to(torch.bfloat16).to(torch.float32) if i < 3 else t for i, t in enumerate(sh))
               for sh in shards]
    for r in range(world):
        got = cea.ulysses_scatter(*shards_v[r], _group(cea, shards_v, r), layout.sizes, heads)
        want = sp_ref.ulysses_scatter(shards, heads, r)
        gotw = cea.ulysses_scatter(*shards_d[r], _group(cea, shards_d, r, torch.bfloat16),
                                   layout.sizes, heads)
        wantw = sp_ref.ulysses_scatter(rounded, heads, r)
        torch.cuda.synchronize()
        for a, b_ in zip(got, want):
            assert torch.equal(a.cpu(), b_)
        for a, b_ in zip(gotw, wantw):
            assert torch.equal(a.cpu(), b_)


def test_ulysses_wire_compression_rules(cea, dev):
    """float16 wire: f32 pieces saturate at 65504 on the way (comm.py:275-282), the positions
    are never compressed, and bf16 activations do not go through an f16 wire at all (same
    width, comm.py:284-290)."""
    world, hq, hkv, D, B, S = 2, 4, 2, 32, 1, 40
    g = torch.Generator().manual_seed(9)
    heads = cea.partition_heads(hq, hkv, world)
    layout = cea.SequenceLayout(S, world, None, "contiguous")
    pos = torch.arange(S).repeat(B, 1)
    for act in (torch.float32, torch.bfloat16):
        q = torch.randn(B, S, hq, D, generator=g).to(act)
        k = torch.randn(B, S, hkv, D, generator=g).to(act)
        v = torch.randn(B, S, hkv, D, generator=g).to(act)
        q[0, ::3, 0, 1] = 1.0e5
        v[0, ::5, 1, 2] = -7.0e4
        shards = [tuple(layout.shard(t, r) for t in (q, k, v, pos)) for r in range(world)]
        shards_d = [tuple(t.to(dev) for t in sh) for sh in shards]
        rounded = [tuple(sp_ref.wire_round(t, torch.float16) for t in sh) for sh in shards]
        for r in range(world):
            got = cea.ulysses_scatter(*shards_d[r], _group(cea, shards_d, r, torch.float16),
                                      layout.sizes, heads)
            want = sp_ref.ulysses_scatter(rounded, heads, r)
            torch.cuda.synchronize()
            for a, b_ in zip(got, want):
                assert torch.equal(a.cpu(), b_), (act, r)
        if act == torch.float32:
            assert rounded[0][0].abs().max().item() == 65504.0
        else:
            assert torch.equal(rounded[0][0], shards[0][0])


def test_ulysses_workload_full_size(cea, dev):
    """The Ulysses workload's shape (65536 tokens, a 64/16-head model over sp=8, D=128,
    bf16): rank 0's scatter equals the head slices of the rank-order concatenation and the
    gather of head outputs equals the rank's token shard, element for element."""
    S, world = 65536, 8
    heads = cea.partition_heads(64, 16, world)
    layout = cea.SequenceLayout(S, world, None, "contiguous")
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(1, S, 64, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(1, S, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, S, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    pos = torch.arange(S, device=dev).view(1, S)
    shards = [tuple(layout.shard(t, r) for t in (q, k, v, pos)) for r in range(world)]
    sh = heads[0]
    q_f, k_f, v_f, pos_f = cea.ulysses_scatter(*shards[0], _group(cea, shards, 0), layout.sizes, heads)
    assert torch.equal(q_f, q[:, :, sh.q_start:sh.q_start + sh.q_count])
    assert torch.equal(k_f, k[:, :, sh.kv_start:sh.kv_start + sh.kv_count])
    assert torch.equal(v_f, v[:, :, sh.kv_start:sh.kv_start + sh.kv_count])
    assert torch.equal(pos_f, pos)
    outs = [q[:, :, h.q_start:h.q_start + h.q_count] for h in heads]
    for r in (0, 5):
        grp = _group(cea, shards, r)
        for j, o in enumerate(outs):
            grp.set_shard(j, out_heads=o)
        got = cea.ulysses_gather(outs[r], grp, layout.sizes, heads)
        assert torch.equal(got, shards[r][0])
    # the head gather of Ulysses decoding (sequence_parallel.py:242-247): every rank's head
    # slice over the same tokens, concatenated along the heads
    grp = _group(cea, shards, 3)
    for j, o in enumerate(outs):
        grp.set_shard(j, out_heads=o)
    assert torch.equal(cea.gather_heads(outs[3], grp, heads), q)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=str)
def test_pack_and_merge_packed_match_oracle(cea, dev, dtype):
    B, Sq, H, Dh = 2, 9, 5, 64
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, Sq, H, Dh, generator=g, dtype=torch.float64).to(dtype)
    k = torch.randn(B, 70, H, Dh, generator=g, dtype=torch.float64).to(dtype)
    v = torch.randn(B, 70, H, Dh, generator=g, dtype=torch.float64).to(dtype)
    qpos = torch.arange(Sq).repeat(B, 1) + 60
    kpos = torch.arange(70).repeat(B, 1)
    kpos[1, 30:] = -1  # partitions 2 and 3 of the second sequence are empty
    cuts = [0, 25, 40, 55, 70]
    parts, parts_ref, outs, lses = [], [], [], []
    gathered = torch.empty(len(cuts) - 1, B, Sq, H, Dh + 1, dtype=dtype, device=dev)
    for i, (a, b_) in enumerate(zip(cuts[:-1], cuts[1:])):
        o, l = cea.attention_with_lse(q.to(dev), k[:, a:b_].to(dev), v[:, a:b_].to(dev),
                                      qpos.to(dev), kpos[:, a:b_].to(dev))
        pk = cea.pack_partial(o, l)
        cea.pack_partial(o, l, gathered[i])
        ro, rl = ref.attention_with_lse(q, k[:, a:b_], v[:, a:b_], qpos, kpos[:, a:b_])
        torch.cuda.synchronize()
        assert torch.equal(pk.cpu(), sp_ref.pack_partial(o.cpu(), l.cpu()))
        assert torch.equal(gathered[i].cpu(), pk.cpu())
        parts.append(pk)
        parts_ref.append(sp_ref.pack_partial(ro, rl))
        outs.append(o)
        lses.append(l)
    mo, ml = cea.merge_packed(gathered, return_lse=True)
    lo, ll = cea.merge_attention_list(outs, lses)
    m16 = cea.merge_packed(parts, out_dtype=torch.bfloat16) if dtype == torch.float32 else None
    want = sp_ref.merge_packed(parts_ref, dtype)
    torch.cuda.synchronize()
    assert torch.equal(mo.cpu(), lo.cpu()) and torch.equal(ml.cpu(), ll.cpu())
    tol = 1e-10 if dtype == torch.float64 else 1e-5 * want.abs().max().item()
    assert (mo.cpu() - want).abs().max().item() <= tol
    if m16 is not None:
        assert m16.dtype == torch.bfloat16 and torch.equal(m16.cpu(), lo.cpu().to(torch.bfloat16))


def test_kv_decode_packed_route_matches_fused(cea, dev):
    """The distributed-KV decode workload (B=32, 32/8 heads, cache 32768, 4 uneven
    partitions) through the packed all-gather route equals the fused single-launch route and
    the oracle on a subset of sequences."""
    w = cea.workloads.kv_decode(device=dev)
    parts = w.partitions()
    group = cea.LocalGroup(len(parts))
    for r, (k, v, p) in enumerate(parts):
        group.set_shard(r, k=k, v=v, pos=p)
    fused = cea.distributed_kv_attention(w.q, *parts[0][:2], w.q_pos, parts[0][2], group)
    packed = cea.distributed_kv_attention_packed(w.q, *parts[0][:2], w.q_pos, parts[0][2], group)
    torch.cuda.synchronize()
    assert packed.dtype == torch.bfloat16 and packed.shape == fused.shape
    assert (packed.float() - fused.float()).abs().max().item() <= 2e-2
    rows = [0, 13, 31]
    wc = cea.workloads.kv_decode(device="cpu", batch=rows)
    ro = sp_ref.distributed_kv_share(wc.q, wc.q_pos, wc.partitions())
    assert (packed[rows].cpu().float() - ro.float()).abs().max().item() <= 2e-2
