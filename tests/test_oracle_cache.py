"""The oracle's KV cache against known answers: growth policy, head-major layout, -1 in
unused position slots, views, and the rotary append (CPU only)."""

from __future__ import annotations

import torch

from oracle import cache_ref as C
from oracle import layers_ref as L


def _block(B, n, H, D, start, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, n, H, D, generator=g)
    v = torch.randn(B, n, H, D, generator=g)
    pos = torch.arange(start, start + n).repeat(B, 1)
    return k, v, pos


def test_growth_sequence_known_answers():
    # capacity = max(needed + reserve, int(1.5 * capacity)) (cache.py:40)
    for reserve, appends, caps in [
        (0, [5, 3, 1, 3, 1], [5, 8, 12, 12, 18]),
        (4, [5, 3, 1, 10], [9, 9, 9, 23]),
        (0, [1, 1, 1, 1, 1, 1], [1, 2, 3, 4, 6, 6]),
    ]:
        c = C.LayerKVCache(reserve)
        t = 0
        got = []
        for n in appends:
            c.append(*_block(2, n, 3, 4, t, t))
            t += n
            got.append(c.capacity)
        assert got == caps, (reserve, got, caps)
        assert c.length == t


def test_layout_views_and_unused_slots():
    c = C.LayerKVCache()
    blocks = [_block(2, n, 3, 8, s, i) for i, (n, s) in enumerate([(4, 0), (2, 4), (5, 6)])]
    for k, v, p in blocks:
        c.append(k, v, p)
    K = torch.cat([b[0] for b in blocks], 1)
    V = torch.cat([b[1] for b in blocks], 1)
    P = torch.cat([b[2] for b in blocks], 1)
    kv, vv, pv = c.view()
    assert torch.equal(kv, K) and torch.equal(vv, V) and torch.equal(pv, P)
    # head-major storage: cache[b, h, t] == block[b, t, h]
    for b in range(2):
        for h in range(3):
            assert torch.equal(c.k[b, h, :11], K[b, :, h])
    assert c.capacity == 11 and bool((c.pos[:, 11:] == -1).all())
    # a grown cache keeps its content and marks the new slots -1
    c.append(*_block(2, 1, 3, 8, 11, 9))
    assert c.capacity == 16 and torch.equal(c.view()[0][:, :11], K)
    assert bool((c.pos[:, 12:] == -1).all())


def test_append_rotary_is_rotation_then_append():
    B, n, H, D = 2, 6, 4, 16
    k, v, pos = _block(B, n, H, D, 3, 1)
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    cos, sin = L.rope_tables(pos, L.inv_freq(D, 1e4), torch.bfloat16)
    a, b = C.LayerKVCache(), C.LayerKVCache()
    a.append_rotary(k, v, pos, cos, sin)
    b.append(L.apply_rotary(k, cos, sin), v, pos)
    assert all(torch.equal(x, y) for x, y in zip(a.view(), b.view()))
    # the rotation of a position-0 token is the identity
    z = C.LayerKVCache()
    p0 = torch.zeros(B, 1, dtype=torch.int64)
    c0, s0 = L.rope_tables(p0, L.inv_freq(D, 1e4), torch.bfloat16)
    z.append_rotary(k[:, :1], v[:, :1], p0, c0, s0)
    assert torch.equal(z.view()[0], k[:, :1])
