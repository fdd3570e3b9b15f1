"""GPU parity of the per-rank sequence-parallel shares and the split-KV decode path.

* ring / Ulysses / distributed-KV on simulated ranks == single-device attention, in f64
  (tests/test_sequence_parallel.py:15-67 of the reference, err < 1e-12 there; 1e-10 here)
  and against the CPU oracle of the same shares in bf16;
* the split-KV decode kernels (short query blocks, cache views, partitions) against the
  oracle's per-partition attention and merge, including each partition's (out, lse).
Tolerances as stated in tests/_cases.py.
"""

import pytest
import torch

from _cases import Case, assert_attention_close, make_positions
from oracle import attention_ref as ref
from oracle import sp_ref

pytestmark = pytest.mark.gpu

B, S, HQ, HKV, D = 2, 13, 6, 3, 4


def _inputs(dtype=torch.float64, d=D, hq=HQ, hkv=HKV, s=S, b=B):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(b, s, hq, d, generator=g, dtype=torch.float64).to(dtype)
    k = torch.randn(b, s, hkv, d, generator=g, dtype=torch.float64).to(dtype)
    v = torch.randn(b, s, hkv, d, generator=g, dtype=torch.float64).to(dtype)
    pos = torch.arange(s).repeat(b, 1)
    pos[1, :3] = -1  # left padding in the second sequence
    pos[1, 3:] -= 3
    return q, k, v, pos


@pytest.mark.parametrize(
    "world,kind,weights,causal",
    [(2, "contiguous", None, True), (2, "zigzag", None, True), (3, "zigzag", [3, 2, 1], True),
     (3, "contiguous", [1, 2, 3], False)],
)
def test_shares_match_single_device_f64(cea, dev, world, kind, weights, causal):
    q, k, v, pos = (t.to(dev) for t in _inputs())
    full = cea.attention.attention(q, k, v, pos, pos, causal=causal)
    valid = (pos >= 0).cpu()
    layout = cea.SequenceLayout(S, world, weights, kind)
    group = cea.LocalGroup(world)
    for r in range(world):
        group.set_shard(r, q=layout.shard(q, r), k=layout.shard(k, r), v=layout.shard(v, r),
                        pos=layout.shard(pos, r))
    ring_parts, uly_parts = [], []
    shards = cea.partition_heads(HQ, HKV, weights or world)
    for r in range(world):
        me = group.view_as(r)
        sh = group.shard(r)
        ring_parts.append(cea.ring_attention(sh["q"], sh["k"], sh["v"], sh["pos"], sh["pos"], me,
                                             layout.sizes, causal=causal))
        out, _ = cea.ulysses_attention(sh["q"], sh["k"], sh["v"], sh["pos"], me, layout.sizes,
                                       shards, causal=causal)
        uly_parts.append(out)
    torch.cuda.synchronize()
    ring = layout.unshard(ring_parts).cpu()
    uly = layout.unshard(uly_parts).cpu()
    assert (ring - full.cpu())[valid].abs().max().item() < 1e-10
    assert (uly - full.cpu())[valid].abs().max().item() < 1e-10
    # decoding: the last two tokens against the sequence-sharded cache
    dkv = cea.distributed_kv_attention(q[:, -2:], group.shard(0)["k"], group.shard(0)["v"],
                                       pos[:, -2:], group.shard(0)["pos"], group, causal=causal)
    torch.cuda.synchronize()
    assert (dkv.cpu() - full.cpu()[:, -2:]).abs().max().item() < 1e-10


def test_ring_share_bf16_matches_oracle(cea, dev):
    """A small zigzag ring share in bf16 against the oracle's ring loop (skip rule, order)."""
    w = cea.workloads.ring_share(seq_len=2048, sp=4, rank=1, hq=8, hkv=2, d=128)
    blocks = [(k.to(dev), v.to(dev), p.to(dev)) for k, v, p in w.blocks]
    group = cea.LocalGroup(4, 1)
    for r, (k, v, p) in enumerate(blocks):
        group.set_shard(r, k=k, v=v, pos=p)
    k1, v1, p1 = blocks[1]
    out, lse = cea.sequence_parallel.ring_attention_with_lse(
        w.q.to(dev), k1, v1, w.q_pos.to(dev), p1, group, w.kv_sizes)
    ro, rl = sp_ref.ring_share(w.q, w.q_pos, w.blocks, 1, with_lse=True)
    torch.cuda.synchronize()
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, "ring share")


@pytest.mark.parametrize("wire", [torch.bfloat16, torch.float16], ids=["bf16-wire", "f16-wire"])
def test_ring_share_with_wire_compression(cea, dev, wire):
    """f64 activations, compressed ring traffic (sequence_parallel.py:101-127, comm.py:275-290):
    blocks from other ranks arrive rounded through the wire dtype (float16 saturating at
    65504), the rank's own block stays at full precision.  Some keys and values exceed the
    float16 range, so the saturation shows in the result.  (f64: keys of magnitude 9e4 make
    scores of a few hundred, whose f32 rounding alone moves the result by ~1e-4 relative
    between any two summation orders; in f64 the comparison is exact to 1e-10.)"""
    world, rank, S, hq, hkv, d = 4, 2, 256, 4, 2, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, S, hq, d, generator=g, dtype=torch.float64) * 0.05
    k = torch.randn(1, S, hkv, d, generator=g, dtype=torch.float64)
    v = torch.randn(1, S, hkv, d, generator=g, dtype=torch.float64)
    k[0, ::17, :, 3] = 9.0e4
    v[0, ::13, :, 5] = -1.0e5
    pos = torch.arange(S).repeat(1, 1)
    layout = cea.SequenceLayout(S, world, None, "zigzag")
    shards = [tuple(layout.shard(t, r) for t in (k, v, pos)) for r in range(world)]
    group = cea.LocalGroup(world, rank, wire_dtype=wire)
    for r, (kr, vr, pr) in enumerate(shards):
        group.set_shard(r, k=kr.to(dev), v=vr.to(dev), pos=pr.to(dev))
    qr, qp = layout.shard(q, rank), layout.shard(pos, rank)
    own = shards[rank]
    out, lse = cea.sequence_parallel.ring_attention_with_lse(
        qr.to(dev), own[0].to(dev), own[1].to(dev), qp.to(dev), own[2].to(dev), group,
        layout.sizes)
    blocks = [(kr, vr, pr) if r == rank else
              (sp_ref.wire_round(kr, wire), sp_ref.wire_round(vr, wire), pr)
              for r, (kr, vr, pr) in enumerate(shards)]
    ro, rl = sp_ref.ring_share(qr, qp, blocks, rank, with_lse=True)
    torch.cuda.synchronize()
    assert_attention_close(out, lse, ro, rl, torch.float64, f"ring share, {wire} wire")
    if wire == torch.float16:  # the unsaturated transfer would differ
        inf_blocks = [(kr, vr, pr) if r == rank else (kr.half().double(), vr.half().double(), pr)
                      for r, (kr, vr, pr) in enumerate(shards)]
        bad, _ = sp_ref.ring_share(qr, qp, inf_blocks, rank, with_lse=True)
        assert not torch.allclose(bad, ro, equal_nan=True)


DECODE_CASES = [
    # (B, Sq, Hq, Hkv, cap, parts, D, kv_map)
    (3, 1, 32, 8, 700, [400, 300], 128, None),
    (2, 1, 8, 8, 1500, [1500], 128, None),
    (2, 2, 8, 4, 999, [333, 333, 333], 128, None),
    (2, 4, 4, 4, 513, [100, 13, 400], 128, None),
    (1, 1, 16, 4, 5000, [2000, 1500, 1000, 500], 128, None),
    # head size 64: the tinyllama-1.1b (32/4) and qwen2-0.5b (14/2) presets
    # (models/config.py:18,21), multi-query with four new tokens
    (3, 1, 32, 4, 700, [400, 300], 64, None),
    (2, 1, 14, 2, 999, [333, 333, 333], 64, None),
    (1, 4, 4, 1, 513, [100, 413], 64, None),
    # explicit maps that are not the h // g grouping: shard 0 of partition_heads(32, 8, 3)
    # (groups of 4, 4, 3; partition.py:141-152) and an arbitrary one
    (2, 2, 11, 3, 800, [500, 300], 128, [0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2]),
    (2, 1, 6, 2, 600, [600], 64, [1, 0, 0, 1, 1, 0]),
]


def _case_id(s):
    return "B{}-Sq{}-H{}/{}-cap{}-p{}-D{}{}".format(*s[:5], len(s[5]), s[6], "-map" if s[7] else "")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
@pytest.mark.parametrize("shape", DECODE_CASES, ids=_case_id)
def test_partitioned_decode_matches_oracle(cea, dev, shape, dtype):
    Bn, Sq, Hq, Hkv, cap, sizes, d, kv_map = shape
    g = torch.Generator().manual_seed(sum(sizes) + Sq + d)
    ck = torch.randn(Bn, Hkv, cap, d, generator=g).to(dtype)
    cv = torch.randn(Bn, Hkv, cap, d, generator=g).to(dtype)
    q = torch.randn(Bn, Sq, Hq, d, generator=g).to(dtype)
    lens = torch.randint(1, cap + 1, (Bn,), generator=g)
    slots = torch.arange(cap).view(1, cap)
    kpos = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
    qpos = (lens - 1).view(-1, 1) + torch.arange(Sq).view(1, Sq) - (Sq - 1)
    qpos = qpos.clamp(min=0)
    ckd, cvd, kpd = ck.to(dev), cv.to(dev), kpos.to(dev)
    parts, parts_cpu, start = [], [], 0
    for n in sizes:
        parts.append((ckd[:, :, start:start + n].transpose(1, 2), cvd[:, :, start:start + n].transpose(1, 2),
                      kpd[:, start:start + n]))
        parts_cpu.append((ck[:, :, start:start + n].transpose(1, 2), cv[:, :, start:start + n].transpose(1, 2),
                          kpos[:, start:start + n]))
        start += n
    out, lse, per = cea.partitioned_attention(q.to(dev), qpos.to(dev), parts, kv_map=kv_map,
                                              return_lse=True, return_parts=True)
    out_q = cea.partitioned_attention(q.to(dev), qpos.to(dev), parts, kv_map=kv_map)
    ro, rl, rparts = sp_ref.distributed_kv_share(q, qpos, parts_cpu, kv_map=kv_map, with_parts=True)
    torch.cuda.synchronize()
    assert out_q.dtype == dtype
    for (po, pl), (qo, ql) in zip(per, rparts):
        assert_attention_close(po, pl, qo, ql, dtype, "partition")
    assert_attention_close(out, lse, ro.float(), rl, dtype, "merged")
    assert (out_q.cpu().float() - ro.float()).abs().max().item() <= 2e-2
    # single-partition attention_with_lse on the decode path
    o1, l1 = cea.attention_with_lse(q.to(dev), *parts[0][:2], qpos.to(dev), parts[0][2], kv_map=kv_map)
    r1, s1 = ref.attention_with_lse(q, *parts_cpu[0][:2], qpos, parts_cpu[0][2], kv_map=kv_map)
    torch.cuda.synchronize()
    assert_attention_close(o1, l1, r1, s1, dtype, "single partition")


@pytest.mark.parametrize("d,kv_map", [(128, None), (64, None), (64, [1, 0, 0, 1, 1, 0])],
                         ids=["d128", "d64", "d64-map"])
def test_partitioned_decode_without_causal_rule(cea, dev, d, kv_map):
    """causal=False with a negative scale on the split-KV decode path: every valid slot is
    visible (k_pos >= 0 alone decides), including slots past the queries' own positions; each
    partition's (out, lse), the merge and the q-dtype result against the oracle."""
    g = torch.Generator().manual_seed(77 + d)
    Bn, Sq, Hq, Hkv, cap, sizes = 3, 2, 6, 2, 900, [500, 250, 150]
    dtype = torch.bfloat16
    ck = torch.randn(Bn, Hkv, cap, d, generator=g).to(dtype)
    cv = torch.randn(Bn, Hkv, cap, d, generator=g).to(dtype)
    q = torch.randn(Bn, Sq, Hq, d, generator=g).to(dtype)
    lens = torch.tensor([900, 321, 17])
    slots = torch.arange(cap).view(1, cap)
    kpos = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
    qpos = torch.tensor([[3, 4], [100, 101], [0, 1]])  # before most of the valid slots
    parts, parts_cpu, start = [], [], 0
    for n in sizes:
        sl = slice(start, start + n)
        parts_cpu.append((ck[:, :, sl].transpose(1, 2), cv[:, :, sl].transpose(1, 2), kpos[:, sl]))
        parts.append(tuple(t.to(dev) for t in parts_cpu[-1]))
        start += n
    kw = dict(causal=False, scale=-0.07, kv_map=kv_map)
    out, lse, per = cea.partitioned_attention(q.to(dev), qpos.to(dev), parts, return_lse=True,
                                              return_parts=True, **kw)
    out_q = cea.partitioned_attention(q.to(dev), qpos.to(dev), parts, **kw)
    torch.cuda.synchronize()
    ro, rl, rparts = sp_ref.distributed_kv_share(q, qpos, parts_cpu, with_parts=True, **kw)
    for i, ((po, pl), (qo, ql)) in enumerate(zip(per, rparts)):
        assert_attention_close(po, pl, qo, ql, dtype, f"partition {i}")
    assert_attention_close(out, lse, ro.float(), rl, dtype, "merged")
    assert out_q.dtype == dtype
    assert (out_q.cpu().float() - ro.float()).abs().max().item() <= 2e-2


def test_kv_decode_workload_subset_matches_oracle(cea, dev):
    """Four sequences of the distributed-KV decode workload (cache 32768, 4 partitions)
    through distributed_kv_attention on simulated ranks vs the oracle."""
    w = cea.workloads.kv_decode(device=dev, batch=[0, 7, 19, 31])
    wc = cea.workloads.kv_decode(device="cpu", batch=[0, 7, 19, 31])
    parts = w.partitions()
    group = cea.LocalGroup(len(parts))
    for r, (k, v, p) in enumerate(parts):
        group.set_shard(r, k=k, v=v, pos=p)
    out = cea.distributed_kv_attention(w.q, parts[0][0], parts[0][1], w.q_pos, parts[0][2], group)
    ro = sp_ref.distributed_kv_share(wc.q, wc.q_pos, wc.partitions())
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    err = (out.cpu().float() - ro.float()).abs().max().item()
    assert err <= 2e-2, err


@pytest.mark.parametrize("wire_kv", [False, True], ids=["fused", "packed"])
def test_distributed_kv_ignores_activation_wire_dtype(cea, dev, wire_kv):
    """Distributed-KV decoding moves no K/V: each rank attends to the partition it stores at
    full precision and only the f32 (out | lse) message is all-gathered, uncompressed
    (sequence_parallel.py:270-279).  With a float16 activation wire and f64 activations whose
    keys / values exceed the float16 range (a rounded or saturated K/V would move the result
    by far more than the f64 tolerance), the result must still be the oracle's."""
    world, B, T, hq, hkv, d = 3, 2, 300, 4, 2, 64
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, 1, hq, d, generator=g, dtype=torch.float64) * 0.01
    k = torch.randn(B, T, hkv, d, generator=g, dtype=torch.float64)
    v = torch.randn(B, T, hkv, d, generator=g, dtype=torch.float64)
    k[:, ::11, :, 2] = 8.0e4
    v[:, ::7, :, 1] = -1.0e5
    pos = torch.arange(T).repeat(B, 1)
    qpos = torch.full((B, 1), T - 1)
    sizes = cea.split_sizes(T, [0.5, 0.3, 0.2])
    group = cea.LocalGroup(world, 1, wire_dtype=torch.float16)
    parts, start = [], 0
    for r, n in enumerate(sizes):
        parts.append((k[:, start:start + n], v[:, start:start + n], pos[:, start:start + n]))
        group.set_shard(r, k=parts[-1][0].to(dev), v=parts[-1][1].to(dev), pos=parts[-1][2].to(dev))
        start += n
    own = [t.to(dev) for t in parts[1]]
    fn = cea.distributed_kv_attention_packed if wire_kv else cea.distributed_kv_attention
    out = fn(q.to(dev), own[0], own[1], qpos.to(dev), own[2], group)
    ro = sp_ref.distributed_kv_share(q, qpos, parts)
    torch.cuda.synchronize()
    assert out.dtype == torch.float64
    err = (out.cpu() - ro).abs().max().item()
    assert err <= 1e-10, err
    # the same K/V rounded through float16 on the way would not pass
    rounded = [(sp_ref.wire_round(kk, torch.float16), sp_ref.wire_round(vv, torch.float16), pp)
               for kk, vv, pp in parts]
    assert (sp_ref.distributed_kv_share(q, qpos, rounded) - ro).abs().max().item() > 1.0


def test_partitioned_fallback_with_many_chunks(cea, dev):
    """Four partitions whose key chunks together exceed what one split-KV launch takes
    (each partition alone would fit): every partition runs as its own attention call inside
    the workspace the library asked for, then the exact merge."""
    B, hq, hkv, d, n = 1, 4, 1, 128, 300_000
    g = torch.Generator().manual_seed(13)
    q = torch.randn(B, 1, hq, d, generator=g).to(torch.bfloat16)
    parts_cpu = []
    for i in range(4):
        k = torch.randn(B, n, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(B, n, hkv, d, generator=g).to(torch.bfloat16)
        p = torch.arange(i * n, (i + 1) * n).view(1, n)
        parts_cpu.append((k, v, p))
    qpos = torch.tensor([[4 * n]])
    parts = [tuple(t.to(dev) for t in pc) for pc in parts_cpu]
    out, lse = cea.partitioned_attention(q.to(dev), qpos.to(dev), parts, return_lse=True)
    ro, rl, _ = sp_ref.distributed_kv_share(q, qpos, parts_cpu, with_parts=True)
    torch.cuda.synchronize()
    assert_attention_close(out, lse, ro.float(), rl, torch.bfloat16, "4 x 300k keys")


def test_partitioned_decode_chunk_pairs_two_tokens(cea, dev):
    """A decode call large enough for the split kernel's chunk pairs (32 rows x 4 kv heads x
    65 chunks of 1024 keys; the last rows take single chunks), with two new tokens per
    sequence (8 query rows per kv head): every partition's (out, lse) and the merged result
    against the oracle on sequences from both kinds of rows.  K / V are drawn on the device;
    only the checked sequences are copied to the host."""
    B, Sq, hq, hkv, d, cap = 32, 2, 16, 4, 128, 65536
    sizes = [39322, cap - 39322]
    g = torch.Generator(device=dev).manual_seed(21)
    ck = torch.randn(B, hkv, cap, d, generator=g, device=dev).to(torch.bfloat16)
    cv = torch.randn(B, hkv, cap, d, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(B, Sq, hq, d, generator=g, device=dev).to(torch.bfloat16)
    gc = torch.Generator().manual_seed(22)
    lens = torch.randint(2, cap + 1, (B,), generator=gc)
    lens[28] = cap  # a full-length sequence among the single-chunk rows
    slots = torch.arange(cap).view(1, cap)
    kpos = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
    qpos = (lens - 2).view(-1, 1) + torch.arange(Sq).view(1, Sq)
    kpd, qpd = kpos.to(dev), qpos.to(dev)
    parts, start = [], 0
    for n in sizes:
        parts.append((ck[:, :, start:start + n].transpose(1, 2), cv[:, :, start:start + n].transpose(1, 2),
                      kpd[:, start:start + n]))
        start += n
    out, lse, per = cea.partitioned_attention(q, qpd, parts, return_lse=True, return_parts=True)
    torch.cuda.synchronize()
    for b in (0, 5, 13, 27, 28, 31):
        sl = slice(b, b + 1)
        pb, start = [], 0
        for n in sizes:
            pb.append((ck[sl, :, start:start + n].transpose(1, 2).cpu(), cv[sl, :, start:start + n].transpose(1, 2).cpu(),
                       kpos[sl, start:start + n]))
            start += n
        ro, rl, rparts = sp_ref.distributed_kv_share(q[sl].cpu(), qpos[sl], pb, with_parts=True)
        for i, ((po, pl), (qo, ql)) in enumerate(zip(per, rparts)):
            assert_attention_close(po[sl], pl[sl], qo, ql, torch.bfloat16, f"seq {b} partition {i}")
        assert_attention_close(out[sl], lse[sl], ro.float(), rl, torch.bfloat16, f"seq {b} merged")


@pytest.mark.parametrize("nranks", [17, 40])
def test_distributed_kv_more_ranks_than_one_launch(cea, dev, nranks):
    """A cache sharded over more ranks than one split-KV launch takes (16): the partitions run
    in groups, each group merged in its reduction, and the groups merged exactly; the result,
    the merged lse and every rank's partial (out, lse) match the oracle's all-at-once merge
    (sequence_parallel.py:273-279 -> attention.py:253-264)."""
    B, hq, hkv, d, cap = 2, 8, 2, 128, 3000
    g = torch.Generator().manual_seed(nranks)
    k = torch.randn(B, cap, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, cap, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(B, 1, hq, d, generator=g).to(torch.bfloat16)
    lens = torch.tensor([cap, 1700])
    slots = torch.arange(cap).view(1, cap)
    pos = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
    qpos = (lens - 1).view(-1, 1)
    sizes = cea.split_sizes(cap, nranks)
    group = cea.LocalGroup(nranks, 3)
    parts_cpu, start = [], 0
    for r, n in enumerate(sizes):
        parts_cpu.append((k[:, start:start + n], v[:, start:start + n], pos[:, start:start + n]))
        group.set_shard(r, k=parts_cpu[-1][0].to(dev), v=parts_cpu[-1][1].to(dev),
                        pos=parts_cpu[-1][2].to(dev))
        start += n
    own = group.shard(3)
    out = cea.distributed_kv_attention(q.to(dev), own["k"], own["v"], qpos.to(dev), own["pos"], group)
    parts = [tuple(group.shard(r)[x] for x in ("k", "v", "pos")) for r in range(nranks)]
    o2, l2, per = cea.partitioned_attention(q.to(dev), qpos.to(dev), parts, return_lse=True,
                                            return_parts=True)
    ro, rl, rparts = sp_ref.distributed_kv_share(q, qpos, parts_cpu, with_parts=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and len(per) == nranks
    assert (out.cpu().float() - ro.float()).abs().max().item() <= 2e-2
    assert_attention_close(o2, l2, ro.float(), rl, torch.bfloat16, f"{nranks} ranks merged")
    for i, ((po, pl), (qo, ql)) in enumerate(zip(per, rparts)):
        assert_attention_close(po, pl, qo, ql, torch.bfloat16, f"rank {i} partial")
