"""GPU parity of a rank's ring-attention share computed in one call (cea_ring_attention).

Every simulated rank's KV block is resident, so ``ring_attention`` hands all of them, in ring
order, to one C-ABI call: bf16 / f16 with head size 64 or 128 and one row stride per call
run as a single prefill launch that carries each query row's softmax state across the blocks;
other calls run block after block into a running (out, lse) pair.  Both routes are checked
against the oracle's ring loop (sequence_parallel.py:94-130: blocks visited in the order
``(rank - step) mod n``, fully hidden blocks skipped, pairwise online merge), with the
tolerances of tests/_cases.py, on the shapes the routes treat differently: uneven blocks whose
last tile is partial, an empty block, padding, no causal mask, irregular and MQA head maps,
``kv_block`` pieces (one call up to 16 pieces, the per-piece loop beyond), blocks with
different row strides (the per-block route) and shares in which no query sees any key.
"""

import pytest
import torch

from _cases import assert_attention_close
from oracle import sp_ref

pytestmark = pytest.mark.gpu


def _share(world, sizes, hq, hkv, d, seed, pad_every=0, dtype=torch.bfloat16, q_len=None):
    """Blocks of ``world`` ranks with ``sizes`` tokens each (positions laid out contiguously
    in rank order, every ``pad_every``-th key padding) and rank 1's queries."""
    g = torch.Generator().manual_seed(seed)
    blocks, start = [], 0
    for s in sizes:
        k = torch.randn(1, s, hkv, d, generator=g).to(dtype)
        v = torch.randn(1, s, hkv, d, generator=g).to(dtype)
        pos = torch.arange(start, start + s).view(1, s)
        if pad_every:
            pos[:, ::pad_every] = -1
        blocks.append((k, v, pos))
        start += s
    rank = 1
    sq = q_len or sizes[rank]
    q = torch.randn(1, sq, hq, d, generator=g).to(dtype)
    q_pos = blocks[rank][2].clone() if q_len is None else torch.arange(start - sq, start).view(1, sq)
    return q, q_pos, blocks, rank


def _group(cea, dev, world, rank, blocks):
    grp = cea.LocalGroup(world, rank)
    for r, (k, v, p) in enumerate(blocks):
        grp.set_shard(r, k=k.to(dev), v=v.to(dev), pos=p.to(dev))
    return grp


def _run(cea, dev, q, q_pos, blocks, rank, **kw):
    grp = _group(cea, dev, len(blocks), rank, blocks)
    own = grp.shard(rank)
    sizes = [b[0].shape[1] for b in blocks]
    out, lse = cea.sequence_parallel.ring_attention_with_lse(
        q.to(dev), own["k"], own["v"], q_pos.to(dev), own["pos"], grp, sizes, **kw)
    plain = cea.ring_attention(q.to(dev), own["k"], own["v"], q_pos.to(dev), own["pos"], grp,
                               sizes, **kw)
    torch.cuda.synchronize()
    return out, lse, plain


CASES = [
    # (world, sizes, hq, hkv, d, pad_every, causal, kv_map, q_len)
    (4, [300, 257, 64, 1000], 8, 2, 128, 0, True, None, None),
    (3, [200, 0, 150], 4, 4, 64, 0, True, None, 120),
    (4, [128, 129, 191, 65], 6, 3, 128, 7, True, None, None),
    (3, [100, 220, 90], 4, 2, 64, 0, False, None, None),
    (4, [96, 160, 33, 250], 6, 2, 128, 0, True, [0, 0, 1, 1, 1, 0], None),
    (2, [300, 300], 8, 1, 128, 5, True, None, None),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "w{}-{}-h{}/{}-d{}-pad{}-{}-{}".format(
    c[0], "_".join(map(str, c[1])), c[2], c[3], c[4], c[5], "causal" if c[6] else "full",
    "map" if c[7] else "reg"))
def test_ring_share_one_call_matches_oracle(cea, dev, case, dtype):
    world, sizes, hq, hkv, d, pad, causal, kv_map, q_len = case
    q, q_pos, blocks, rank = _share(world, sizes, hq, hkv, d, seed=len(sizes) + hq, pad_every=pad,
                                    dtype=dtype, q_len=q_len)
    out, lse, plain = _run(cea, dev, q, q_pos, blocks, rank, causal=causal, kv_map=kv_map)
    ro, rl = sp_ref.ring_share(q, q_pos, blocks, rank, causal=causal, kv_map=kv_map, with_lse=True)
    assert_attention_close(out, lse, ro, rl, dtype, "ring share (out, lse)")
    assert plain.dtype == dtype
    # the plain call writes the result in q's dtype in the kernel: the f32 result rounded once
    assert torch.equal(plain.cpu(), out.to(dtype).cpu())


@pytest.mark.parametrize("kv_block,expect_loop", [(100, False), (16, True)], ids=["pieces", "loop"])
def test_ring_share_kv_block(cea, dev, kv_block, expect_loop):
    """kv_block splits every block into pieces (attention.py:225-236): up to 16 pieces are one
    call, more run piece after piece; both give the oracle's blockwise result."""
    q, q_pos, blocks, rank = _share(3, [200, 190, 60], 4, 2, 64, seed=3)
    n_pieces = sum(-(-b[0].shape[1] // kv_block) for b in blocks)
    assert (n_pieces > cea._native.MAX_PARTS) == expect_loop
    out, lse, plain = _run(cea, dev, q, q_pos, blocks, rank, kv_block=kv_block)
    ro, rl = sp_ref.ring_share(q, q_pos, blocks, rank, kv_block=kv_block, with_lse=True)
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, f"ring share, kv_block {kv_block}")
    assert_attention_close(plain.float(), None, ro.to(torch.bfloat16).float(), None, torch.bfloat16,
                           "ring share, q dtype")


def test_ring_share_blocks_with_different_row_strides(cea, dev):
    """A block that is a view with another row stride (a head slice of a wider tensor) sends
    the call down the per-block route; the result is the same function."""
    q, q_pos, blocks, rank = _share(3, [130, 140, 70], 4, 2, 128, seed=11)
    wide = torch.randn(1, 70, 4, 128).to(torch.bfloat16)
    wide[:, :, :2] = blocks[2][0]
    wide_v = torch.randn(1, 70, 4, 128).to(torch.bfloat16)
    wide_v[:, :, :2] = blocks[2][1]
    grp = _group(cea, dev, 3, rank, blocks)
    grp.set_shard(2, k=wide.to(dev)[:, :, :2], v=wide_v.to(dev)[:, :, :2])
    own = grp.shard(rank)
    out, lse = cea.sequence_parallel.ring_attention_with_lse(
        q.to(dev), own["k"], own["v"], q_pos.to(dev), own["pos"], grp, [130, 140, 70])
    torch.cuda.synchronize()
    ro, rl = sp_ref.ring_share(q, q_pos, blocks, rank, with_lse=True)
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, "ring share, strided block")


def test_ring_share_nothing_visible(cea, dev):
    """Queries before every key under the causal rule, and all-padding keys: zeros in q's
    dtype (sequence_parallel.py:128-129), lse -inf."""
    q, _, blocks, rank = _share(3, [64, 80, 90], 4, 2, 128, seed=2)
    q_pos = torch.full((1, 80), -5)
    out, lse, plain = _run(cea, dev, q, q_pos, blocks, rank)
    assert plain.dtype == torch.bfloat16 and not plain.cpu().any()
    assert not out.cpu().any() and (lse.cpu() == float("-inf")).all()
    pad_blocks = [(k, v, torch.full_like(p, -1)) for k, v, p in blocks]
    q_pos = blocks[rank][2]
    out, lse, plain = _run(cea, dev, q, q_pos, pad_blocks, rank)
    assert not plain.cpu().any() and (lse.cpu() == float("-inf")).all()


def test_ring_share_batch_of_two(cea, dev):
    """Two batch rows with different padding in every block (the tile summaries are per batch
    row): the one-call share against the oracle's ring loop."""
    g = torch.Generator().manual_seed(21)
    sizes, hq, hkv, d = [260, 200, 130], 4, 2, 128
    blocks, start = [], 0
    for n in sizes:
        k = torch.randn(2, n, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(2, n, hkv, d, generator=g).to(torch.bfloat16)
        pos = torch.arange(start, start + n).repeat(2, 1)
        pos[1, n // 3:] = -1  # the second row is padded from a third of each block on
        blocks.append((k, v, pos))
        start += n
    rank = 1
    q = torch.randn(2, sizes[rank], hq, d, generator=g).to(torch.bfloat16)
    q_pos = blocks[rank][2].clone()
    q_pos[1] = torch.arange(sizes[0], sizes[0] + sizes[rank])
    out, lse, plain = _run(cea, dev, q, q_pos, blocks, rank)
    ro, rl = sp_ref.ring_share(q, q_pos, blocks, rank, with_lse=True)
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, "ring share, two batch rows")
    assert torch.equal(plain.cpu(), out.to(torch.bfloat16).cpu())


@pytest.mark.parametrize("sizes", [[0, 0, 0], [0, 90, 0]], ids=["all-empty", "one-block"])
def test_ring_share_empty_blocks(cea, dev, sizes):
    """Ranks holding no keys: with no key anywhere the share is the merge's neutral element
    (zeros, lse -inf); with one non-empty block it is that block's attention."""
    g = torch.Generator().manual_seed(31)
    hq, hkv, d = 4, 2, 128
    blocks, start = [], 0
    for n in sizes:
        blocks.append((torch.randn(1, n, hkv, d, generator=g).to(torch.bfloat16),
                       torch.randn(1, n, hkv, d, generator=g).to(torch.bfloat16),
                       torch.arange(start, start + n).view(1, n)))
        start += n
    q = torch.randn(1, 50, hq, d, generator=g).to(torch.bfloat16)
    q_pos = torch.arange(40, 90).view(1, 50)
    out, lse, plain = _run(cea, dev, q, q_pos, blocks, 1)
    assert torch.equal(plain.cpu(), out.to(torch.bfloat16).cpu())
    ro, rl = sp_ref.ring_share(q, q_pos, blocks, 1, with_lse=True)
    if rl is None:  # the reference skips every block and returns zeros (no lse)
        assert not out.cpu().any() and (lse.cpu() == float("-inf")).all()
        assert not ro.any()
    else:
        assert_attention_close(out, lse, ro, rl, torch.bfloat16, f"ring share {sizes}")


def test_ring_share_no_queries(cea, dev):
    """A rank with no query tokens returns empty results of the right shapes."""
    q, q_pos, blocks, rank = _share(3, [100, 120, 80], 4, 2, 64, seed=5)
    q, q_pos = q[:, :0], q_pos[:, :0]
    out, lse, plain = _run(cea, dev, q, q_pos, blocks, rank)
    assert out.shape == (1, 0, 4, 64) and lse.shape == (1, 4, 0) and plain.shape == (1, 0, 4, 64)


def test_ring_share_rejects_a_block_off_the_device(cea, dev):
    """Every tensor of a call must live on the queries' device: a value block left on the
    host raises before any kernel runs."""
    q, q_pos, blocks, rank = _share(3, [100, 120, 80], 4, 2, 64, seed=9)
    grp = _group(cea, dev, 3, rank, blocks)
    k2, v2, p2 = blocks[2]
    grp.set_shard(2, k=k2.to(dev), v=v2, pos=p2.to(dev))  # v stays on the host
    own = grp.shard(rank)
    with pytest.raises(RuntimeError):
        cea.ring_attention(q.to(dev), own["k"], own["v"], q_pos.to(dev), own["pos"], grp,
                           [100, 120, 80])
