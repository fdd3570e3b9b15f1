"""HIP-graph capture of the operators.

* Replays of captured ring-share, distributed-KV decode, key-split prefill and layer-op calls
  equal the eager results on every replay, with eager work on the device between the
  replays (the kernels write every scratch value they read in the same call and record no
  memset).
* The operator library's per-stream workspace: a buffer that a capture recorded stays
  allocated when a later, larger call on that stream replaces it, so replays never write into
  memory the allocator has handed out again.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _attn_inputs(dev, s, seed, hq=4, hkv=2, d=128):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, s, hq, d, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, s, hkv, d, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(1, s, hkv, d, generator=g).to(torch.bfloat16).to(dev)
    pos = torch.arange(s).view(1, s).to(dev)
    return q, k, v, pos


def test_captured_workspace_survives_growth(cea, dev):
    s = torch.cuda.Stream(dev)
    q, k, v, pos = _attn_inputs(dev, 256, 1)
    bq, bk, bv, bpos = _attn_inputs(dev, 16384, 2)  # 256 tiles: a larger workspace
    with torch.cuda.stream(s):
        ref_o, ref_l = cea.attention_with_lse(q, k, v, pos, pos)  # the stream's first workspace
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out, lse = cea.attention_with_lse(q, k, v, pos, pos)
    with torch.cuda.stream(s):
        cea.attention_with_lse(bq, bk, bv, bpos, bpos)  # replaces the captured workspace
        fillers = [torch.full((4096,), 7, dtype=torch.uint8, device=dev) for _ in range(32)]
    s.synchronize()
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o) and torch.equal(lse, ref_l), f"replay {i}"
        assert all(bool((f == 7).all()) for f in fillers), f"replay {i} wrote into reused memory"
        with torch.cuda.stream(s):
            cea.attention_with_lse(bq, bk, bv, bpos, bpos)
        s.synchronize()


def _replays_match(fn, eager_work, n=3):
    """Captures fn() (a tuple of tensors), replays it n times with eager_work() between the
    replays, and checks every replay against the eager result."""
    ref = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    for i in range(n):
        for t in outs:
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, ref):
            assert torch.equal(a, b), f"replay {i}"
        eager_work()
        torch.cuda.synchronize()


def test_ring_share_replays(cea, dev):
    g = torch.Generator().manual_seed(3)
    sizes, hq, hkv, d = [300, 257, 64, 1000], 8, 2, 128
    group, start = cea.LocalGroup(len(sizes), 1), 0
    for r, n in enumerate(sizes):
        k = torch.randn(1, n, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn(1, n, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        group.set_shard(r, k=k, v=v, pos=torch.arange(start, start + n).view(1, n).to(dev))
        start += n
    own = group.shard(1)
    q = torch.randn(1, sizes[1], hq, d, generator=g).to(torch.bfloat16).to(dev)

    def share():
        out, lse = cea.sequence_parallel.ring_attention_with_lse(
            q, own["k"], own["v"], own["pos"], own["pos"], group, sizes)
        plain = cea.ring_attention(q, own["k"], own["v"], own["pos"], own["pos"], group, sizes)
        return out, lse, plain

    bq, bk, bv, bpos = _attn_inputs(dev, 4096, 4)
    _replays_match(share, lambda: cea.attention_with_lse(bq, bk, bv, bpos, bpos))


def test_distributed_kv_decode_replays(cea, dev):
    w = cea.workloads.kv_decode(device=dev, batch=[0, 5, 9, 30], cap=4096, min_len=64)
    parts = w.partitions()

    def step():
        out, lse = cea.partitioned_attention(w.q, w.q_pos, parts, return_lse=True)
        return out, lse, cea.partitioned_attention(w.q, w.q_pos, parts)

    bq, bk, bv, bpos = _attn_inputs(dev, 2048, 5)
    _replays_match(step, lambda: cea.attention_with_lse(bq, bk, bv, bpos, bpos))


def test_layer_ops_replays(cea, dev):
    g = torch.Generator().manual_seed(6)
    x = torch.randn(64, 1024, generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.02 * torch.randn(1024, generator=g)).to(torch.bfloat16).to(dev)
    pos = torch.arange(64).to(dev)
    inv = cea.layers.rope_inv_freq(128, 10000.0).to(dev)
    gate = torch.randn(64, 2048, generator=g).to(torch.bfloat16).to(dev)
    up = torch.randn(64, 2048, generator=g).to(torch.bfloat16).to(dev)

    def step():
        y = cea.rmsnorm_rope(x, w, 1e-5, pos, inv, 8)
        h = cea.gated_mul(gate, up, "silu")
        return y, h

    _replays_match(step, lambda: cea.gated_mul(up, gate, "gelu"))


def test_key_split_and_subgroup_decode_replays(cea, dev):
    """A prefill chunk that takes the key-split route (partials in the workspace, then the
    list merge) and a decode step with 32 query heads on one KV head (sub-group units)."""
    q, k, v, pos = _attn_inputs(dev, 6000, 7, hq=8, hkv=2)
    qc, qpc = q[:, -96:], pos[:, -96:]
    g = torch.Generator().manual_seed(8)
    dq = torch.randn(2, 1, 32, 128, generator=g).to(torch.bfloat16).to(dev)
    dk = torch.randn(2, 3000, 1, 128, generator=g).to(torch.bfloat16).to(dev)
    dv = torch.randn(2, 3000, 1, 128, generator=g).to(torch.bfloat16).to(dev)
    dkp = torch.arange(3000).repeat(2, 1).to(dev)
    dqp = torch.full((2, 1), 2999).to(dev)

    def step():
        out, lse = cea.attention_with_lse(qc, k, v, qpc, pos)
        plain = cea.attention.attention(qc, k, v, qpc, pos)
        dout, dlse = cea.attention_with_lse(dq, dk, dv, dqp, dkp)
        return out, lse, plain, dout, dlse

    bq, bk, bv, bpos = _attn_inputs(dev, 2048, 9)
    _replays_match(step, lambda: cea.attention_with_lse(bq, bk, bv, bpos, bpos))
