"""Seeded random sweep of attention calls against the oracle, on the GPU.

Combinations the hand-picked cases do not pin one by one: batch, query and key counts
(partial tiles, one-row blocks), head counts with regular and irregular kv maps, head sizes
of the matrix-core, f32 and generic kernels, every mask pattern of tests/_cases.py, causal
and not, default / negative / small scales, kv_block splits, and partitioned (distributed-KV)
calls with 1 to 5 partitions of random sizes through the split-KV decode route, and ring
shares over 2 to 5 simulated ranks through the one-call route (empty and tiny blocks,
padding, two batch rows, head sizes 64 and 128, regular and irregular maps), and short query blocks against long key blocks
(key splits, query heads packed per workgroup, decode units of part of a group).  The cases
are drawn from a fixed seed, so a run is reproducible; tolerances are those of
tests/_cases.py.
"""

from __future__ import annotations

import random

import pytest
import torch

from _cases import Case, assert_attention_close
from oracle import attention_ref as ref
from oracle import sp_ref

pytestmark = pytest.mark.gpu


def _attention_cases(n=160, seed=20261202):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        D = rng.choice([64, 128, 128, 64, 96, 32])
        Hkv = rng.choice([1, 2, 3, 4])
        G = rng.choice([1, 2, 4])
        Hq = Hkv * G
        kv_map = None
        if rng.random() < 0.2:  # irregular grouping (every kv head used at least once)
            heads = list(range(Hkv)) + [rng.randrange(Hkv) for _ in range(Hq - Hkv)]
            rng.shuffle(heads)
            kv_map = tuple(heads)
        kind = rng.choice(["aligned", "left_pad", "right_pad", "zigzag", "decode", "random",
                           "random", "all_pad"])
        B = rng.choice([1, 2, 3])
        if kind in ("aligned", "left_pad", "right_pad"):
            Sq = Sk = rng.choice([1, 2, 31, 64, 65, 127, 200, 257, 301])
            if kind == "left_pad":
                Sq = Sk = max(Sq, 4)
        elif kind == "decode":
            Sq, Sk = rng.choice([1, 1, 2, 3, 4]), rng.choice([5, 64, 300, 1000, 2049])
        else:
            Sq, Sk = rng.choice([1, 3, 33, 100, 250]), rng.choice([1, 16, 65, 200, 777, 1500])
            if kind == "zigzag":
                Sq = max(Sq, 2)
        causal = kind in ("aligned", "left_pad", "right_pad", "decode") or rng.random() < 0.5
        scale = rng.choice([None, None, None, -0.07, 0.02, 1.3])
        cases.append(Case(B, Sq, Sk, Hq, Hkv, D, kind, causal, kv_map, scale, seed=i))
    return cases


ATTN = _attention_cases()


@pytest.mark.parametrize("case", ATTN, ids=str)
def test_random_attention_matches_oracle(cea, dev, case):
    """One random case, in the half-precision dtype its head size runs on the matrix cores
    (bf16 or f16, chosen by the case seed) and in f32; with a kv_block split for every
    third case."""
    dtypes = [torch.bfloat16 if case.seed % 2 == 0 else torch.float16, torch.float32]
    kv_block = None
    if case.seed % 3 == 0 and case.Sk > 1:
        kv_block = max(1, case.Sk // random.Random(case.seed).choice([2, 3, 5]))
    for dtype in dtypes:
        q, k, v, qp, kp = case.tensors(dtype)
        print(f"case {case} {dtype} kv_block={kv_block}", flush=True)
        out, lse = cea.attention_with_lse(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev),
                                          causal=case.causal, scale=case.scale,
                                          kv_map=case.kv_map, kv_block=kv_block)
        torch.cuda.synchronize()
        # torch's CPU flash operator (the reference's CPU route) applies its causal mask before
        # the scale, so a negative scale turns masked scores into +inf and rows into NaN; the
        # math route evaluates the defined softmax(scale * q.k) there
        route = "math" if case.scale is not None and case.scale <= 0 else "flash"
        ro, rl = ref.attention_with_lse(q, k, v, qp, kp, causal=case.causal, scale=case.scale,
                                        kv_map=case.kv_map, kv_block=kv_block, route=route)
        assert_attention_close(out, lse, ro, rl, dtype, f"{case} {dtype}")


def _long_key_cases(n=80, seed=9090):
    """Short query blocks against long key blocks: the key-split prefill launches, query
    heads packed 2-8 to a workgroup, and decode units of part of a KV head's group (up to 32
    query heads per KV head)."""
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        D = rng.choice([64, 128])
        Hkv = rng.choice([1, 2, 4])
        G = rng.choice([1, 2, 4, 8, 16, 32])
        Hq = Hkv * G
        Sk = rng.choice([1500, 3000, 5000, 9000, 17000])
        Sq = rng.choice([1, 2, 3, 5, 17, 40, 100, 130, 200])
        while Sq * Sk * Hq > 60_000_000 and Sq > 1:  # keeps the oracle at about a second
            Sq //= 2
        kind = rng.choice(["decode", "random", "right_pad", "chunk", "chunk"])
        causal = kind != "random" or rng.random() < 0.5
        scale = rng.choice([None, None, -0.05, 0.3])
        cases.append((rng.choice([1, 1, 2]), Sq, Sk, Hq, Hkv, D, kind, causal, scale, i))
    return cases


def _long_key_tensors(B, Sq, Sk, Hq, Hkv, D, kind, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    kp = torch.arange(Sk).repeat(B, 1)
    end = torch.full((B,), Sk)
    if kind == "right_pad":  # valid keys end early; rows past the end are padding too
        end = torch.randint(Sq, Sk + 1, (B,), generator=g)
        kp = torch.where(kp < end.view(-1, 1), kp, torch.full_like(kp, -1))
    if kind == "random":
        qp = torch.randint(0, Sk, (B, Sq), generator=g)
    else:  # the last Sq valid positions (a chunk at the end, or decode tokens)
        qp = end.view(-1, 1) - Sq + torch.arange(Sq).view(1, Sq)
    return q, k, v, qp, kp


LONG = _long_key_cases()


@pytest.mark.parametrize("lc", LONG, ids=lambda c: "B{}-Sq{}-Sk{}-H{}/{}-D{}-{}-{}-s{}".format(
    *c[:6], c[6], "c" if c[7] else "nc", c[8]))
def test_random_short_queries_long_keys(cea, dev, lc):
    B, Sq, Sk, Hq, Hkv, D, kind, causal, scale, seed = lc
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    q, k, v, qp, kp = _long_key_tensors(B, Sq, Sk, Hq, Hkv, D, kind, seed, dtype)
    print(f"long-key case {lc} {dtype}", flush=True)
    out, lse = cea.attention_with_lse(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev),
                                      causal=causal, scale=scale)
    plain = cea.attention.attention(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev),
                                    causal=causal, scale=scale)
    torch.cuda.synchronize()
    route = "math" if scale is not None and scale <= 0 else "flash"
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp, causal=causal, scale=scale, route=route)
    assert_attention_close(out, lse, ro, rl, dtype, str(lc))
    assert plain.dtype == dtype
    assert (plain.cpu().double() - ro.double()).abs().max().item() <= 2e-2, str(lc)


def _partition_cases(n=48, seed=7177):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        nparts = rng.randint(1, 5)
        sizes = [rng.choice([1, 17, 256, 700, 1024, 1500, 3000]) for _ in range(nparts)]
        Sq = rng.choice([1, 1, 2, 4])
        G = rng.choice([1, 2, 4])
        if Sq * G > 16:
            G = 16 // Sq
        Hkv = rng.choice([1, 2, 4])
        cases.append((i, rng.choice([1, 2, 5]), Sq, Hkv * G, Hkv, sizes,
                      rng.choice([torch.bfloat16, torch.float16])))
    return cases


@pytest.mark.parametrize("pc", _partition_cases(), ids=lambda c: f"p{c[0]}-B{c[1]}-Sq{c[2]}-H{c[3]}/{c[4]}-{c[5]}")
def test_random_partitions_match_oracle(cea, dev, pc):
    """partitioned_attention over 1-5 KV partitions of random sizes (about a tenth of the
    slots invalid, -1; the last Sq positions as causal queries) against the oracle's
    distributed-KV share: each partition's (out, lse), the merge and the q-dtype result."""
    i, B, Sq, Hq, Hkv, sizes, dtype = pc
    D = 128
    g = torch.Generator().manual_seed(1000 + i)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
    parts, start = [], 0
    for n in sizes:
        k = torch.randn(B, n, Hkv, D, generator=g).to(dtype)
        v = torch.randn(B, n, Hkv, D, generator=g).to(dtype)
        pos = (torch.arange(n) + start).repeat(B, 1)
        drop = torch.rand(B, n, generator=g) < 0.1  # invalid slots (-1)
        pos[drop] = -1
        parts.append((k, v, pos))
        start += n
    q_pos = (start - Sq + torch.arange(Sq)).repeat(B, 1)
    print(f"partitions {sizes} B{B} Sq{Sq} H{Hq}/{Hkv} {dtype}", flush=True)
    pd = [(k.to(dev), v.to(dev), p.to(dev)) for k, v, p in parts]
    out, lse, per = cea.partitioned_attention(q.to(dev), q_pos.to(dev), pd, return_lse=True,
                                              return_parts=True)
    plain = cea.partitioned_attention(q.to(dev), q_pos.to(dev), pd)
    torch.cuda.synchronize()
    rb, rl, partial = sp_ref.distributed_kv_share(q, q_pos, parts, with_parts=True)
    for j, ((po, pl), (ro, rlp)) in enumerate(zip(per, partial)):
        assert_attention_close(po, pl, ro, rlp, dtype, f"partition {j}")
    ro = partial[0][0] if len(partial) == 1 else ref.merge_many([x[0] for x in partial],
                                                                 [x[1] for x in partial])[0]
    assert_attention_close(out, lse, ro, rl, dtype, "merged")
    assert plain.dtype == dtype
    assert (plain.float().cpu() - rb.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("sizes", [[0, 700, 0, 1500], [0, 0], [1024, 0], [0, 3000, 17]],
                         ids=lambda s: "-".join(map(str, s)))
def test_partitions_with_empty_ranks(cea, dev, sizes):
    """Ranks holding no KV yet: an empty partition's attention_with_lse is (0, -inf)
    (attention.py:152-157) and merges as the identity; with every partition empty the result
    is (0, -inf) throughout."""
    B, Sq, Hq, Hkv, D, dtype = 2, 1, 8, 2, 128, torch.bfloat16
    g = torch.Generator().manual_seed(sum(sizes) + len(sizes))
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
    parts, start = [], 0
    for n in sizes:
        parts.append((torch.randn(B, n, Hkv, D, generator=g).to(dtype),
                      torch.randn(B, n, Hkv, D, generator=g).to(dtype),
                      (torch.arange(n) + start).repeat(B, 1)))
        start += n
    q_pos = torch.full((B, Sq), max(start - 1, 0))
    print(f"partitions {sizes}", flush=True)
    pd = [(k.to(dev), v.to(dev), p.to(dev)) for k, v, p in parts]
    out, lse, per = cea.partitioned_attention(q.to(dev), q_pos.to(dev), pd, return_lse=True,
                                              return_parts=True)
    torch.cuda.synchronize()
    rb, rl, partial = sp_ref.distributed_kv_share(q, q_pos, parts, with_parts=True)
    for j, ((po, pl), (ro, rlp)) in enumerate(zip(per, partial)):
        assert_attention_close(po, pl, ro, rlp, dtype, f"partition {j}")
    ro = partial[0][0] if len(partial) == 1 else ref.merge_many([x[0] for x in partial],
                                                                 [x[1] for x in partial])[0]
    assert_attention_close(out, lse, ro, rl, dtype, "merged")
    if start == 0:
        assert bool((out == 0).all()) and bool(torch.isinf(lse).all())


def _ring_cases(n=40, seed=4242):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        world = rng.choice([2, 3, 4, 5])
        sizes = [rng.choice([0, rng.randrange(1, 80), rng.randrange(64, 700)]) for _ in range(world)]
        rank = rng.randrange(world)
        if sizes[rank] == 0:
            sizes[rank] = rng.randrange(1, 300)
        hkv = rng.choice([1, 2, 4])
        hq = hkv * rng.choice([1, 2, 3, 4])
        kv_map = None
        if rng.random() < 0.25:
            heads = list(range(hkv)) + [rng.randrange(hkv) for _ in range(hq - hkv)]
            kv_map = tuple(sorted(heads))
        causal = rng.random() < 0.7
        # non-positive scales only without the causal rule (the CPU flash operator returns
        # NaN for is_causal with scale <= 0)
        scale = rng.choice([None, None, 0.05] + ([] if causal else [-0.1]))
        cases.append((i, world, rank, rng.choice([1, 1, 2]), sizes, hq, hkv, rng.choice([64, 128]),
                      rng.choice([torch.bfloat16, torch.float16]), causal, kv_map, scale,
                      rng.random() < 0.3))
    return cases


@pytest.mark.parametrize("rc", _ring_cases(), ids=lambda c: f"r{c[0]}-w{c[1]}-{c[4]}")
def test_random_ring_shares_match_oracle(cea, dev, rc):
    """One rank's ring share in one call (cea_ring_attention) against the oracle's ring loop:
    (out, lse) and the q-dtype result (the f32 result rounded once)."""
    i, world, rank, B, sizes, hq, hkv, d, dtype, causal, kv_map, scale, padded = rc
    g = torch.Generator().manual_seed(5000 + i)
    blocks, start = [], 0
    for n in sizes:
        k = torch.randn(B, n, hkv, d, generator=g).to(dtype)
        v = torch.randn(B, n, hkv, d, generator=g).to(dtype)
        pos = torch.arange(start, start + n).repeat(B, 1)
        if padded and n:
            pos[torch.rand(B, n, generator=g) < 0.2] = -1
        blocks.append((k, v, pos))
        start += n
    q = torch.randn(B, sizes[rank], hq, d, generator=g).to(dtype)
    q_pos = blocks[rank][2].clone()
    print(f"ring w{world} r{rank} B{B} {sizes} h{hq}/{hkv} d{d} {dtype} causal={causal} "
          f"map={kv_map} scale={scale}", flush=True)
    grp = cea.LocalGroup(world, rank)
    for r, (k, v, p) in enumerate(blocks):
        grp.set_shard(r, k=k.to(dev), v=v.to(dev), pos=p.to(dev))
    own = grp.shard(rank)
    kw = dict(causal=causal, scale=scale, kv_map=kv_map)
    out, lse = cea.sequence_parallel.ring_attention_with_lse(q.to(dev), own["k"], own["v"],
                                                             q_pos.to(dev), own["pos"], grp, sizes, **kw)
    plain = cea.ring_attention(q.to(dev), own["k"], own["v"], q_pos.to(dev), own["pos"], grp, sizes, **kw)
    torch.cuda.synchronize()
    ro, rl = sp_ref.ring_share(q, q_pos, blocks, rank, with_lse=True, **kw)
    if rl is None:  # no block visible to any query: zeros (the reference returns no lse)
        assert not out.cpu().any() and (lse.cpu() == float("-inf")).all()
    else:
        assert_attention_close(out, lse, ro, rl, dtype, "ring share")
    assert torch.equal(plain.cpu(), out.to(dtype).cpu())
