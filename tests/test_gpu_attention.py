"""GPU parity of attention_with_lse / attention / merges against the CPU oracle.

Every case runs the gfx950 kernels through the C ABI (via the package's ctypes binding)
and compares with oracle.attention_ref on bit-identical inputs; tolerances are stated in
tests/_cases.py.  The bf16/f16 cases with D in {64, 128} run the MFMA prefill kernel, the
others the generic kernel.
"""

import math

import pytest
import torch

from _cases import Case, assert_attention_close
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

CASES = [
    # reference known-answer shapes (tests/test_attention.py)
    Case(2, 7, 7, 4, 4, 8, "aligned", True),
    Case(2, 7, 7, 4, 4, 8, "aligned", False),
    Case(1, 9, 9, 6, 2, 4, "aligned", True),
    Case(1, 9, 9, 6, 2, 4, "aligned", True, kv_map=(0, 0, 0, 1, 1, 1)),
    Case(1, 4, 4, 2, 2, 4, "left_pad", True),
    Case(1, 3, 3, 1, 1, 16, "aligned", True),
    # masks, maps and scales on the MFMA head sizes
    Case(2, 130, 130, 8, 2, 128, "aligned", True),
    Case(2, 130, 130, 8, 2, 128, "left_pad", True),
    Case(1, 200, 200, 4, 4, 128, "right_pad", True),
    Case(1, 150, 96, 8, 2, 128, "zigzag", True),
    Case(3, 1, 300, 8, 2, 128, "decode", True),
    Case(2, 70, 190, 4, 1, 64, "random", True),
    Case(2, 70, 190, 4, 2, 64, "random", False),
    Case(1, 64, 64, 4, 3, 128, "aligned", True, kv_map=(0, 2, 1, 1)),
    Case(1, 100, 100, 2, 2, 64, "aligned", True, scale=-0.05),
    Case(1, 100, 100, 2, 2, 64, "aligned", True, scale=0.0),
    Case(1, 33, 65, 2, 1, 128, "all_pad", True),
    Case(1, 257, 257, 2, 1, 96, "aligned", True),
    # odd key counts (partial last tile), pipelines of many tiles, several list passes
    Case(2, 97, 131, 8, 2, 128, "random", True),
    Case(1, 131, 131, 4, 1, 128, "left_pad", True),
    Case(1, 257, 257, 8, 8, 64, "aligned", True),
    Case(1, 700, 700, 2, 1, 128, "aligned", True),
    Case(2, 300, 777, 4, 2, 128, "random", False),
    Case(1, 2, 140001, 2, 1, 64, "decode", True),
]

DTYPES = [torch.float64, torch.float32, torch.bfloat16, torch.float16]


def _ids(c):
    return str(c)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_attention_with_lse_matches_oracle(cea, dev, case, dtype):
    q, k, v, qp, kp = case.tensors(dtype)
    out, lse = cea.attention_with_lse(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev),
                                      causal=case.causal, scale=case.scale, kv_map=case.kv_map)
    # torch's CPU flash operator returns NaN for scale <= 0; the math route evaluates the
    # defined softmax(scale * q.k) there (and is exact in f64)
    route = "math" if dtype == torch.float64 or (case.scale is not None and case.scale <= 0) else "flash"
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp, causal=case.causal, scale=case.scale,
                                    kv_map=case.kv_map, route=route)
    torch.cuda.synchronize()
    assert out.dtype == ref.acc_dtype(dtype) and lse.dtype == ref.acc_dtype(dtype)
    assert_attention_close(out, lse, ro, rl, dtype, str(case))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["float32", "bfloat16"])
@pytest.mark.parametrize("case", [CASES[0], CASES[6], CASES[9], CASES[11]], ids=_ids)
def test_plain_attention_matches_oracle(cea, dev, case, dtype):
    q, k, v, qp, kp = case.tensors(dtype)
    out = cea.attention.attention(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev),
                                  causal=case.causal, kv_map=case.kv_map)
    ro = ref.plain_attention(q, k, v, qp, kp, causal=case.causal, kv_map=case.kv_map)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    err = (out.cpu().double() - ro.double()).abs().max().item()
    if dtype == torch.float32:
        err /= ro.abs().max().item()
    assert err <= tol, err


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_split_kv_merged_equals_unsplit(cea, dev, dtype):
    """Merged disjoint key sets == full attention (tests/test_attention.py:37-49), through
    merge_attention_list, chained merge_attention and the in-epilogue online merge."""
    case = Case(2, 96, 160, 8, 2, 128 if dtype in (torch.bfloat16, torch.float16) else 16,
                "aligned" if False else "random", True, seed=7)
    q, k, v, qp, kp = case.tensors(dtype)
    qd, kd, vd, qpd, kpd = (t.to(dev) for t in (q, k, v, qp, kp))
    full, full_lse = cea.attention_with_lse(qd, kd, vd, qpd, kpd)
    idx = torch.randperm(case.Sk, generator=torch.Generator().manual_seed(0))
    parts = [idx[:30], idx[30:101], idx[101:]]
    res = [cea.attention_with_lse(qd, kd[:, p.to(dev)], vd[:, p.to(dev)], qpd, kpd[:, p.to(dev)])
           for p in parts]
    out, lse = cea.merge_attention_list([r[0] for r in res], [r[1] for r in res])
    o2, l2 = cea.merge_attention(*cea.merge_attention(res[0][0], res[0][1], res[1][0], res[1][1]),
                                 res[2][0], res[2][1])
    acc = ref.acc_dtype(dtype)
    o3 = torch.zeros_like(full)
    l3 = torch.full_like(full_lse, float("-inf"))
    for p in parts:
        cea.attention_with_lse_into(o3, l3, qd, kd[:, p.to(dev)], vd[:, p.to(dev)], qpd, kpd[:, p.to(dev)])
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp, route="math" if dtype == torch.float64 else "flash")
    torch.cuda.synchronize()
    for o, l, name in ((out, lse, "list"), (o2, l2, "pairwise"), (o3, l3, "online")):
        assert o.dtype == acc
        assert_attention_close(o, l, full, full_lse, dtype, name)
        assert_attention_close(o, l, ro, rl, dtype, name + " vs oracle")


def test_merge_with_empty_partial_is_identity(cea, dev):
    """tests/test_attention.py:52-63: padded rows are (0, -inf); merging an empty partial
    (Sk = 0) changes nothing."""
    case = Case(1, 4, 4, 2, 2, 4, "left_pad", True, seed=10)
    q, k, v, qp, kp = case.tensors(torch.float64)
    qd, kd, vd, qpd, kpd = (t.to(dev) for t in (q, k, v, qp, kp))
    out, lse = cea.attention_with_lse(qd, kd, vd, qpd, kpd)
    assert torch.isfinite(out).all()
    empty_o, empty_l = cea.attention_with_lse(qd, kd[:, :0], vd[:, :0], qpd, kpd[:, :0])
    merged, mlse = cea.merge_attention(out, lse, empty_o, empty_l)
    torch.cuda.synchronize()
    assert torch.equal(merged.cpu(), out.cpu())
    assert torch.equal(mlse.cpu(), lse.cpu())


def test_default_scale(cea, dev):
    case = Case(1, 3, 3, 1, 1, 16, "aligned", True, seed=13)
    q, k, v, qp, kp = (t.to(dev) for t in case.tensors(torch.float64))
    a = cea.attention.attention(q, k, v, qp, kp)
    b = cea.attention.attention(q, k, v, qp, kp, scale=1 / math.sqrt(16))
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bfloat16", "float32"])
def test_head_major_cache_views_and_kv_block(cea, dev, dtype):
    """Token-major views of a head-major [B, H, cap, D] cache (models/cache.py:64-74) are read
    in place; kv_block gives the same result as one block (attention.py:225-236)."""
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, cap, D, T = 2, 8, 2, 300, 128, 257
    ck = torch.randn(B, Hkv, cap, D, generator=g).to(dtype)
    cv = torch.randn(B, Hkv, cap, D, generator=g).to(dtype)
    q = torch.randn(B, 5, Hq, D, generator=g).to(dtype)
    kpos = torch.arange(T).repeat(B, 1)
    qpos = torch.arange(T - 5, T).repeat(B, 1)
    kview = ck[:, :, :T].transpose(1, 2)
    vview = cv[:, :, :T].transpose(1, 2)
    ckd, cvd = ck.to(dev), cv.to(dev)
    kd, vd = ckd[:, :, :T].transpose(1, 2), cvd[:, :, :T].transpose(1, 2)
    assert not kd.is_contiguous()
    out, lse = cea.attention_with_lse(q.to(dev), kd, vd, qpos.to(dev), kpos.to(dev))
    ob, lb = cea.attention_with_lse(q.to(dev), kd, vd, qpos.to(dev), kpos.to(dev), kv_block=64)
    ro, rl = ref.attention_with_lse(q, kview, vview, qpos, kpos)
    torch.cuda.synchronize()
    assert_attention_close(out, lse, ro, rl, dtype, "cache view")
    assert_attention_close(ob, lb, ro, rl, dtype, "cache view kv_block")


@pytest.mark.parametrize("dtype,Sq,D,final_f32",
                         [(torch.bfloat16, 300, 128, False), (torch.bfloat16, 300, 128, True),
                          (torch.float16, 200, 64, False), (torch.float32, 40, 64, False),
                          (torch.bfloat16, 1, 128, False), (torch.bfloat16, 100, 96, False)],
                         ids=["bf16-mfma", "bf16-mfma-f32out", "f16-mfma", "f32-generic",
                              "bf16-decode", "bf16-generic-d96"])
def test_merge_final_equals_merge_then_cast(cea, dev, dtype, Sq, D, final_f32):
    """The last ring merge with the cast fused (cea_attention_merge_final) returns exactly
    merge-then-cast, on the MFMA kernel and on the kernels that fall back to a separate cast;
    an empty block casts the running pair."""
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, Sk = 2, 4, 2, 230
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype).to(dev)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype).to(dev)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype).to(dev)
    qpos = (torch.arange(Sq) + 150).repeat(B, 1).to(dev)
    kpos = torch.arange(Sk).repeat(B, 1)
    kpos[1, 200:] = -1
    kpos = kpos.to(dev)
    out = torch.zeros(B, Sq, Hq, D, device=dev)
    lse = torch.full((B, Hq, Sq), float("-inf"), device=dev)
    cea.attention_with_lse_into(out, lse, q, k[:, :100], v[:, :100], qpos, kpos[:, :100])
    out2, lse2 = out.clone(), lse.clone()
    cea.attention_with_lse_into(out2, lse2, q, k[:, 100:], v[:, 100:], qpos, kpos[:, 100:])
    fdt = torch.float32 if final_f32 else dtype
    final = torch.empty(B, Sq, Hq, D, dtype=fdt, device=dev)
    lse3 = lse.clone()
    cea.attention_with_lse_into(out.clone(), lse3, q, k[:, 100:], v[:, 100:], qpos, kpos[:, 100:],
                                final=final)
    empty = torch.empty(B, Sq, Hq, D, dtype=fdt, device=dev)
    lse4 = lse2.clone()
    cea.attention_with_lse_into(out2.clone(), lse4, q, k[:, :0], v[:, :0], qpos, kpos[:, :0],
                                final=empty)
    torch.cuda.synchronize()
    assert torch.equal(final, out2.to(fdt))
    assert torch.equal(lse3, lse2)
    assert torch.equal(empty, out2.to(fdt)) and torch.equal(lse4, lse2)


def test_ring_attention_fused_cast_is_exact(cea, dev):
    """ring_attention's last step writes the bf16 result in its epilogue: equal, bit for bit,
    to the f32 merged output of ring_attention_with_lse cast to bf16, for the ring workload's
    layout at reduced length (sp=4 zigzag, GQA 8/2, D=128)."""
    w = cea.workloads.ring_share(device=dev, seq_len=4096, hq=8, hkv=2)
    comm = cea.LocalGroup(w.layout.num_ranks, w.rank)
    for r, (k, v, p) in enumerate(w.blocks):
        comm.set_shard(r, k=k, v=v, pos=p)
    k0, v0, p0 = w.blocks[w.rank]
    res = cea.ring_attention(w.q, k0, v0, w.q_pos, p0, comm, w.kv_sizes)
    o, _ = cea.sequence_parallel.ring_attention_with_lse(w.q, k0, v0, w.q_pos, p0, comm, w.kv_sizes)
    torch.cuda.synchronize()
    assert res.dtype == torch.bfloat16
    assert torch.equal(res, o.to(torch.bfloat16))


@pytest.mark.parametrize("D", [64, 128])
def test_f32_matrix_core_and_generic_paths(cea, dev, D):
    """f32 inputs with 16-byte aligned rows run the f32 matrix-core kernel; a view whose rows
    start 4 bytes off alignment runs the generic kernel.  Both against the oracle (rel 1e-5),
    with odd query / key counts (partial 16-row and 16-key tiles), GQA, right padding, the
    in-place merge of a second key block, and a one-row (decode-shaped) query."""
    g = torch.Generator().manual_seed(D)
    B, Sq, Sk, Hq, Hkv = 2, 45, 333, 8, 2
    q = torch.randn(B, Sq, Hq, D + 1, generator=g)
    k = torch.randn(B, Sk, Hkv, D + 1, generator=g)
    v = torch.randn(B, Sk, Hkv, D + 1, generator=g)
    kp = torch.arange(Sk).repeat(B, 1)
    kp[1, -40:] = -1
    qp = torch.arange(Sk - Sq, Sk).repeat(B, 1)
    ro, rl = ref.attention_with_lse(q[..., :D], k[..., :D], v[..., :D], qp, kp)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    for name, sl in (("aligned", slice(0, D)), ("offset", slice(1, D + 1))):
        if name == "aligned":  # contiguous copies: 16-byte aligned rows
            qa, ka, va = qd[..., sl].contiguous(), kd[..., sl].contiguous(), vd[..., sl].contiguous()
            r_o, r_l = ro, rl
        else:
            qa, ka, va = qd[..., sl], kd[..., sl], vd[..., sl]
            r_o, r_l = ref.attention_with_lse(q[..., sl], k[..., sl], v[..., sl], qp, kp)
        out, lse = cea.attention_with_lse(qa, ka, va, qp.to(dev), kp.to(dev))
        torch.cuda.synchronize()
        assert_attention_close(out, lse, r_o, r_l, torch.float32, f"f32 D{D} {name}")
    # running merge of two key blocks == one call
    qa, ka, va = qd[..., :D].contiguous(), kd[..., :D].contiguous(), vd[..., :D].contiguous()
    o2 = torch.zeros(B, Sq, Hq, D, device=dev)
    l2 = torch.full((B, Hq, Sq), float("-inf"), device=dev)
    for lo, hi in ((0, 150), (150, Sk)):
        cea.attention_with_lse_into(o2, l2, qa, ka[:, lo:hi], va[:, lo:hi], qp.to(dev), kp[:, lo:hi].to(dev))
    torch.cuda.synchronize()
    assert_attention_close(o2, l2, ro, rl, torch.float32, f"f32 D{D} merged blocks")
    # one query row per sequence
    o1, l1 = cea.attention_with_lse(qa[:, -1:], ka, va, qp[:, -1:].to(dev), kp.to(dev))
    torch.cuda.synchronize()
    assert_attention_close(o1, l1, ro[:, -1:], rl[:, :, -1:], torch.float32, f"f32 D{D} decode row")


@pytest.mark.parametrize("Sq,Sk", [(5, 0), (0, 7), (0, 0)])
def test_empty_query_or_key_block(cea, dev, Sq, Sk):
    """No query rows or no keys: the reference's early empty result (attention.py:152-157),
    out zeros and lse -inf of the accumulation dtype (plain attention: zeros of q's dtype)."""
    g = torch.Generator().manual_seed(Sq * 10 + Sk)
    q = torch.randn(2, Sq, 4, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(2, Sk, 2, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, Sk, 2, 128, generator=g).to(torch.bfloat16)
    qp, kp = torch.arange(Sq).repeat(2, 1), torch.arange(Sk).repeat(2, 1)
    out, lse = cea.attention_with_lse(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev))
    plain = cea.attention.attention(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev))
    torch.cuda.synchronize()
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp)
    assert out.shape == ro.shape and out.dtype == ro.dtype and lse.shape == rl.shape
    assert torch.equal(out.cpu(), ro) and torch.equal(lse.cpu(), rl)
    assert plain.shape == q.shape and plain.dtype == q.dtype and bool((plain == 0).all())


def test_key_block_spanning_more_than_4gib(cea, dev):
    """K and V as strided views whose rows are 1 MiB apart, so one (batch, KV head) block spans
    more than 4 GiB: the matrix-core prefill kernel addresses every tile from a 64-bit base
    with 32-bit offsets inside the tile, so the call is bit-identical to the same call on
    contiguous copies (the route those take) and within the bf16 tolerances of the oracle;
    the same for a decode-shaped call and for a one-launch ring share over two such blocks."""
    g = torch.Generator().manual_seed(11)
    B, Sq, Sk, hq, hkv, d = 1, 300, 4160, 4, 2, 128
    row = 1 << 19  # elements per key row of the storage (1 MiB of bf16)
    q = torch.randn(B, Sq, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Sk, hkv, d, generator=g).to(torch.bfloat16)
    kp = torch.arange(Sk).view(1, Sk)
    qp = torch.arange(Sk - Sq, Sk).view(1, Sq)
    views = []
    for t in (k, v):
        store = torch.empty(Sk, row, dtype=torch.bfloat16, device=dev)
        store[:, :hkv * d] = t.view(Sk, hkv * d).to(dev)
        views.append(store[:, :hkv * d].view(1, Sk, hkv, d))
    kv, vv = views
    assert kv.stride(1) * 2 * (Sk - 1) > 1 << 32
    qd, kd, vd, qpd, kpd = q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev)
    out, lse = cea.attention_with_lse(qd, kv, vv, qpd, kpd)
    ref_o, ref_l = cea.attention_with_lse(qd, kd, vd, qpd, kpd)
    dout, dlse = cea.attention_with_lse(qd[:, -1:], kv, vv, qpd[:, -1:], kpd)
    dref_o, dref_l = cea.attention_with_lse(qd[:, -1:], kd, vd, qpd[:, -1:], kpd)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(lse, ref_l)
    assert torch.equal(dout, dref_o) and torch.equal(dlse, dref_l)
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp)
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, "block beyond 4 GiB")
    # a ring share over two blocks of the strided storage, in one launch
    n = Sk // 2
    sizes = [n, Sk - n]
    results = []
    for kk, vv_ in ((kv, vv), (kd, vd)):
        comm = cea.LocalGroup(2, 1)
        for r, (lo, hi) in enumerate(((0, n), (n, Sk))):
            comm.set_shard(r, k=kk[:, lo:hi], v=vv_[:, lo:hi], pos=kpd[:, lo:hi])
        own = comm.shard(1)
        results.append(cea.sequence_parallel.ring_attention_with_lse(
            qd, own["k"], own["v"], qpd, own["pos"], comm, sizes))
    torch.cuda.synchronize()
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
    assert_attention_close(results[0][0], results[0][1], ro, rl, torch.bfloat16, "ring beyond 4 GiB")


def test_decode_against_more_than_a_million_keys(cea, dev):
    """A decode-shaped call against 1.2 M keys (2344 chunks of the split-KV kernels) and a
    distributed-KV step over four partitions of 300 k keys each, both single split-KV
    launches: against the oracle at the bf16 tolerances.  One key near the end of the range
    is planted to dominate head 0's softmax, so a dropped chunk changes the output, not only
    the lse."""
    g = torch.Generator().manual_seed(12)
    Sk, hq, hkv, d = 1_200_000, 4, 1, 64
    q = torch.randn(1, 1, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, Sk, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(1, Sk, hkv, d, generator=g).to(torch.bfloat16)
    k[0, 1_100_000, 0] = 4 * q[0, 0, 0]
    kp = torch.arange(Sk).view(1, Sk)
    kp[0, -1000:] = -1
    qp = torch.tensor([[Sk - 500]])
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp)
    qd, kd, vd, qpd, kpd = q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev)
    out, lse = cea.attention_with_lse(qd, kd, vd, qpd, kpd)
    torch.cuda.synchronize()
    assert ro[0, 0, 0].sub(v[0, 1_100_000, 0].double()).abs().max() < 1e-2  # the planted key rules
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, "decode over 1.2 M keys")
    cuts = [0, 300_000, 600_000, 900_000, Sk]
    parts = [(kd[:, a:b], vd[:, a:b], kpd[:, a:b]) for a, b in zip(cuts, cuts[1:])]
    pout, plse = cea.partitioned_attention(qd, qpd, parts, return_lse=True)
    torch.cuda.synchronize()
    assert_attention_close(pout, plse, ro, rl, torch.bfloat16, "four partitions of 300 k keys")


@pytest.mark.parametrize("shape", [(3, 1, 5000, 32, 1, 128), (2, 2, 3000, 16, 1, 64),
                                   (2, 3, 4000, 24, 4, 128)],
                         ids=["mqa-g32", "g16-two-tokens", "g6-three-tokens"])
def test_decode_with_more_rows_per_kv_head_than_a_unit(cea, dev, shape):
    """Decode shapes whose query rows per KV head (Sq x G) exceed the 16 a split-KV unit
    takes run one unit per query head, each reading its KV head's tiles: against the oracle,
    with a -1-tailed cache per sequence."""
    B, Sq, Sk, Hq, Hkv, D = shape
    g = torch.Generator().manual_seed(Sk)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16)
    lens = torch.randint(Sq, Sk + 1, (B,), generator=g)
    slots = torch.arange(Sk).view(1, Sk)
    kp = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
    qp = lens.view(-1, 1) - Sq + torch.arange(Sq).view(1, Sq)
    ro, rl = ref.attention_with_lse(q, k, v, qp, kp)
    out, lse = cea.attention_with_lse(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev))
    plain = cea.attention.attention(q.to(dev), k.to(dev), v.to(dev), qp.to(dev), kp.to(dev))
    torch.cuda.synchronize()
    assert_attention_close(out, lse, ro, rl, torch.bfloat16, str(shape))
    assert (plain.cpu().double() - ro.double()).abs().max().item() <= 2e-2
