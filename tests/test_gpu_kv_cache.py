"""GPU parity of the KV-cache append kernel (cea_kv_append) through the C ABI.

The kernel's result must equal the oracle's LayerKVCache (cache.py semantics) after
apply_rotary, bit for bit: the rotation is three separately rounded tensor ops in both (no
transcendental inside: the tables are an input), and the append is a copy.  Covered: a
growth sequence of appends, strided k/v (column slices of a fused QKV projection output),
tables broadcast over the batch, bf16/f16/f32/f64, the plain append, a full-size append of
one rank's 8192-token prefill (GQA 8 KV heads, D=128), and the argument checks.
"""

from __future__ import annotations

import pytest
import torch

from oracle import cache_ref as C
from oracle import layers_ref as L

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _same(gpu_cache, ref_cache):
    kg, vg, pg = (t.cpu() for t in gpu_cache.view())
    kr, vr, pr = ref_cache.view()
    assert torch.equal(kg, kr), (kg - kr).abs().max().item()
    assert torch.equal(vg, vr)
    assert torch.equal(pg, pr)
    assert gpu_cache.capacity == ref_cache.capacity
    assert bool((gpu_cache.pos[:, gpu_cache.length:] == -1).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
def test_append_rotary_growth_sequence(cea, dev, dtype):
    B, H, D = 2, 4, 128
    inv = L.inv_freq(D, 1e4, dtype=torch.float64 if dtype == torch.float64 else torch.float32)
    gc, rc = cea.LayerKVCache(reserve=3), C.LayerKVCache(reserve=3)
    t = 0
    for i, n in enumerate([5, 3, 1, 7, 16, 2]):
        g = _gen(i)
        k = torch.randn(B, n, H, D, generator=g).to(dtype)
        v = torch.randn(B, n, H, D, generator=g).to(dtype)
        pos = torch.arange(t, t + n).repeat(B, 1)
        pos[1] += 100  # a second sequence at other positions
        cos, sin = L.rope_tables(pos, inv, dtype)
        gc.append_rotary(k.to(dev), v.to(dev), pos.to(dev), cos.to(dev), sin.to(dev))
        rc.append_rotary(k, v, pos, cos, sin)
        t += n
    torch.cuda.synchronize()
    _same(gc, rc)


def test_strided_qkv_slices_and_broadcast_tables(cea, dev):
    """k, v as column slices of one fused QKV output [B, n, (Hq + 2 Hkv) D] (llama.py:196,
    205), tables [1, n, D] broadcast over the batch."""
    B, n, Hq, Hkv, D = 3, 33, 8, 2, 64
    fused = torch.randn(B, n, (Hq + 2 * Hkv) * D, generator=_gen(7)).to(torch.bfloat16)
    k = fused[:, :, Hq * D:(Hq + Hkv) * D].view(B, n, Hkv, D)
    v = fused[:, :, (Hq + Hkv) * D:].view(B, n, Hkv, D)
    pos = torch.arange(n).repeat(B, 1)
    cos, sin = L.rope_tables(pos[:1], L.inv_freq(D, 5e5), torch.bfloat16)
    fd = fused.to(dev)
    kd = fd[:, :, Hq * D:(Hq + Hkv) * D].view(B, n, Hkv, D)
    vd = fd[:, :, (Hq + Hkv) * D:].view(B, n, Hkv, D)
    gc, rc = cea.LayerKVCache(), C.LayerKVCache()
    gc.append_rotary(kd, vd, pos.to(dev), cos.to(dev), sin.to(dev))
    rc.append_rotary(k, v, pos, cos.expand(B, n, D), sin.expand(B, n, D))
    torch.cuda.synchronize()
    _same(gc, rc)


def test_plain_append_and_decode_steps(cea, dev):
    """Prefill of 40 tokens then 5 single-token decode appends (llama.py:252-255), no
    rotation: an exact copy into the head-major layout."""
    B, H, D = 4, 8, 128
    gc, rc = cea.LayerKVCache(), C.LayerKVCache()
    for i, n in enumerate([40, 1, 1, 1, 1, 1]):
        g = _gen(20 + i)
        k = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
        v = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
        pos = torch.arange(gc.length, gc.length + n).repeat(B, 1)
        gc.append(k.to(dev), v.to(dev), pos.to(dev))
        rc.append(k, v, pos)
    torch.cuda.synchronize()
    _same(gc, rc)


def test_full_size_prefill_append(cea, dev):
    """One rank's 8192-token chunk, 8 KV heads, D=128, bf16, into a cache that already holds
    1000 tokens (slots 1000..9191)."""
    B, n, H, D = 1, 8192, 8, 128
    g = _gen(31)
    k0 = torch.randn(B, 1000, H, D, generator=g).to(torch.bfloat16)
    v0 = torch.randn(B, 1000, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
    p0 = torch.arange(1000).view(1, -1)
    pos = torch.arange(1000, 1000 + n).view(1, -1)
    cos, sin = L.rope_tables(pos, L.inv_freq(D, 1e4), torch.bfloat16)
    gc, rc = cea.LayerKVCache(), C.LayerKVCache()
    gc.append(k0.to(dev), v0.to(dev), p0.to(dev))
    rc.append(k0, v0, p0)
    gc.append_rotary(k.to(dev), v.to(dev), pos.to(dev), cos.to(dev), sin.to(dev))
    rc.append_rotary(k, v, pos, cos, sin)
    torch.cuda.synchronize()
    _same(gc, rc)


def test_kv_append_argument_errors(cea, dev):
    k = torch.randn(1, 4, 2, 8, device=dev)
    ck = torch.zeros(1, 2, 6, 8, device=dev)
    cp = torch.full((1, 6), -1, dtype=torch.int64, device=dev)
    pos = torch.arange(4, device=dev).view(1, 4)
    cea.kv_append(ck, ck.clone(), cp, 0, k, k, pos)
    with pytest.raises(ValueError):  # slots 4..7 exceed the capacity 6
        cea.kv_append(ck, ck.clone(), cp, 4, k, k, pos)
    with pytest.raises(ValueError):  # cache head count differs
        cea.kv_append(torch.zeros(1, 3, 6, 8, device=dev), torch.zeros(1, 3, 6, 8, device=dev),
                      cp, 0, k, k, pos)
    with pytest.raises(ValueError):  # only one table
        cea.kv_append(ck, ck.clone(), cp, 0, k, k, pos, torch.ones(1, 4, 8, device=dev), None)
    with pytest.raises(RuntimeError):  # host tensors are refused, never computed on the CPU
        cea.kv_append(ck.cpu(), ck.cpu(), cp.cpu(), 0, k.cpu(), k.cpu(), pos.cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_values_with_their_own_heads_and_size(cea, dev, dtype):
    """V with another head count and head size than K (cache.py:42-43 sizes V from V): the
    cache keeps V in an allocation of its own; K is rotated by the rotary kernel; the cached
    tensors equal the oracle's bit for bit through a growth sequence of rotary and plain
    appends."""
    B, Hk, Dk, Hv, Dv = 2, 4, 64, 2, 96
    inv = L.inv_freq(Dk, 1e4, dtype=torch.float32)
    gc, rc = cea.LayerKVCache(reserve=2), C.LayerKVCache(reserve=2)
    t = 0
    for i, n in enumerate([4, 9, 1, 20]):
        g = _gen(40 + i)
        k = torch.randn(B, n, Hk, Dk, generator=g).to(dtype)
        v = torch.randn(B, n, Hv, Dv, generator=g).to(dtype)
        pos = torch.arange(t, t + n).repeat(B, 1)
        if i % 2 == 0:
            cos, sin = L.rope_tables(pos, inv, dtype)
            gc.append_rotary(k.to(dev), v.to(dev), pos.to(dev), cos.to(dev), sin.to(dev))
            rc.append_rotary(k, v, pos, cos, sin)
        else:
            gc.append(k.to(dev), v.to(dev), pos.to(dev))
            rc.append(k, v, pos)
        t += n
    torch.cuda.synchronize()
    assert tuple(gc.v.shape[1::2]) == (Hv, Dv) and tuple(gc.k.shape[1::2]) == (Hk, Dk)
    _same(gc, rc)
    assert gc.nbytes() == B * t * (Hk * Dk + Hv * Dv) * torch.empty(0, dtype=dtype).element_size()
    assert gc.capacity >= t + 2  # the next append fits: the shape check, not a regrowth, refuses it
    with pytest.raises(ValueError):  # a later V of yet another shape
        gc.append(torch.zeros(B, 2, Hk, Dk, dtype=dtype, device=dev),
                  torch.zeros(B, 2, Hv, Dk, dtype=dtype, device=dev),
                  torch.arange(t, t + 2).repeat(B, 1).to(dev))
