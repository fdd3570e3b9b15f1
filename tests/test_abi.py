"""The C ABI library: it loads, exports every function include/collab_edge_attn.h declares,
and rejects inconsistent arguments with the documented status codes before any device work
(argument validation only: no kernel runs here)."""

import ctypes
import subprocess

import pytest
import torch

from conftest import PKG


def test_header_lists_the_entry_points(cea):
    names = cea._native.header_symbols()
    for expected in ("cea_attention_with_lse", "cea_merge_attention", "cea_merge_attention_list",
                     "cea_partitioned_attention", "cea_rmsnorm", "cea_rope_tables",
                     "cea_apply_rotary", "cea_rmsnorm_rope", "cea_silu_mul", "cea_linear",
                     "cea_linear_gated", "cea_last_error"):
        assert expected in names


def test_library_loads_and_exports_every_header_symbol(cea):
    lib_path = cea._native.LIB_PATH
    assert lib_path.exists(), "build the library first (__graft_entry__.build())"
    raw = ctypes.CDLL(str(lib_path))  # fails on unresolved symbols (RTLD_NOW semantics below)
    for name in cea._native.header_symbols():
        assert hasattr(raw, name), f"{name} declared in the header but not exported"
    # every undefined symbol must come from a system / ROCm library, never from our own code
    out = subprocess.run(["nm", "-D", "--undefined-only", str(lib_path)], capture_output=True, text=True)
    own = [l for l in out.stdout.splitlines() if "cea" in l]
    assert not own, f"unresolved library-internal symbols: {own}"


def test_version(cea):
    assert cea._native.load_library().cea_version() >= 100


def _t(shape, dtype_code, data=0x1000):
    a = cea_tensor = None
    import importlib

    nat = importlib.import_module(PKG + "._native")
    a = nat.CeaTensor()
    a.data = data
    a.dtype = dtype_code
    a.ndim = len(shape)
    stride = 1
    for i in reversed(range(len(shape))):
        a.size[i] = shape[i]
        a.stride[i] = stride
        stride *= shape[i]
    return a


def test_attention_rejects_bad_shapes_without_launching(cea):
    nat = cea._native
    lib = nat.load_library()
    bf16, i64, f32 = 1, 4, 0
    q = _t((1, 4, 4, 8), bf16)
    k = _t((1, 5, 3, 8), bf16)   # 4 query heads cannot share 3 KV heads evenly
    v = _t((1, 5, 3, 8), bf16)
    qp, kp = _t((1, 4), i64), _t((1, 5), i64)
    out, lse = _t((1, 4, 4, 8), f32), _t((1, 4, 4), f32)
    rc = lib.cea_attention_with_lse(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), ctypes.byref(qp),
                                    ctypes.byref(kp), 1, 0.125, None, 0, ctypes.byref(out),
                                    ctypes.byref(lse), 0, None, 0, None)
    assert rc == nat.EINVAL
    assert "cannot share" in nat.last_error()
    with pytest.raises(ValueError, match="cannot share"):
        nat.check(rc, "attention_with_lse")
    # explicit map of the wrong length
    arr = (ctypes.c_int32 * 3)(0, 1, 2)
    rc = lib.cea_attention_with_lse(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), ctypes.byref(qp),
                                    ctypes.byref(kp), 1, 0.125, arr, 3, ctypes.byref(out),
                                    ctypes.byref(lse), 0, None, 0, None)
    assert rc == nat.EINVAL and "one entry per query head" in nat.last_error()
    # lse of the wrong shape
    bad_lse = _t((1, 4, 5), f32)
    k2, v2 = _t((1, 5, 2, 8), bf16), _t((1, 5, 2, 8), bf16)
    rc = lib.cea_attention_with_lse(ctypes.byref(q), ctypes.byref(k2), ctypes.byref(v2), ctypes.byref(qp),
                                    ctypes.byref(kp), 1, 0.125, None, 0, ctypes.byref(out),
                                    ctypes.byref(bad_lse), 0, None, 0, None)
    assert rc == nat.EINVAL and "lse must be" in nat.last_error()


def test_merge_rejects_too_many_parts_and_bad_dtypes(cea):
    nat = cea._native
    lib = nat.load_library()
    outs = (nat.CeaTensor * 17)(*[_t((1, 2, 2, 4), 0) for _ in range(17)])
    lses = (nat.CeaTensor * 17)(*[_t((1, 2, 2), 0) for _ in range(17)])
    o, l = _t((1, 2, 2, 4), 0), _t((1, 2, 2), 0)
    rc = lib.cea_merge_attention_list(17, outs, lses, ctypes.byref(o), ctypes.byref(l), None)
    assert rc == nat.EUNSUPPORTED
    b = (nat.CeaTensor * 2)(_t((1, 2, 2, 4), 1), _t((1, 2, 2, 4), 1))
    rc = lib.cea_merge_attention_list(2, b, lses, ctypes.byref(o), ctypes.byref(l), None)
    assert rc == nat.EUNSUPPORTED and "float32 or float64" in nat.last_error()


def test_layer_ops_reject_bad_shapes(cea):
    nat = cea._native
    lib = nat.load_library()
    x, w, y = _t((4, 8), 1), _t((7,), 1), _t((4, 8), 1)
    rc = lib.cea_rmsnorm(ctypes.byref(x), ctypes.byref(w), 1e-5, ctypes.byref(y), None)
    assert rc == nat.EINVAL and "weight" in nat.last_error()
    x4 = _t((1, 2, 2, 7), 1)
    cs = _t((1, 2, 7), 1)
    rc = lib.cea_apply_rotary(ctypes.byref(x4), ctypes.byref(cs), ctypes.byref(cs), ctypes.byref(x4), None)
    assert rc == nat.EINVAL and "even" in nat.last_error()
    g, u = _t((4, 8), 1), _t((4, 9), 1)
    rc = lib.cea_silu_mul(ctypes.byref(g), ctypes.byref(u), ctypes.byref(g), None)
    assert rc == nat.EINVAL


def test_projection_rejects_bad_arguments(cea):
    """cea_linear / cea_linear_gated validate shapes, dtypes and the activation before any
    launch (the pointers here are never dereferenced)."""
    nat = cea._native
    lib = nat.load_library()
    bf16, i64 = 1, 4
    x, w, y = _t((4, 8), bf16), _t((5, 7), bf16), _t((4, 5), bf16)
    rc = lib.cea_linear(ctypes.byref(x), ctypes.byref(w), None, ctypes.byref(y), None)
    assert rc == nat.EINVAL and "input features" in nat.last_error()
    w = _t((5, 8), bf16)
    b = _t((4,), bf16)
    rc = lib.cea_linear(ctypes.byref(x), ctypes.byref(w), ctypes.byref(b), ctypes.byref(y), None)
    assert rc == nat.EINVAL and "bias" in nat.last_error()
    y6 = _t((4, 6), bf16)
    rc = lib.cea_linear(ctypes.byref(x), ctypes.byref(w), None, ctypes.byref(y6), None)
    assert rc == nat.EINVAL and "y must be" in nat.last_error()
    xi, wi, yi = _t((4, 8), i64), _t((5, 8), i64), _t((4, 5), i64)
    rc = lib.cea_linear(ctypes.byref(xi), ctypes.byref(wi), None, ctypes.byref(yi), None)
    assert rc == nat.EUNSUPPORTED
    wu = _t((6, 8), bf16)
    rc = lib.cea_linear_gated(ctypes.byref(x), ctypes.byref(w), ctypes.byref(wu), None, None,
                              ctypes.byref(y), 0, None)
    assert rc == nat.EINVAL and "same number of rows" in nat.last_error()
    rc = lib.cea_linear_gated(ctypes.byref(x), ctypes.byref(w), ctypes.byref(w), None, None,
                              ctypes.byref(y), 9, None)
    assert rc == nat.EUNSUPPORTED and "activation" in nat.last_error()
    bg = _t((5,), bf16)
    rc = lib.cea_linear_gated(ctypes.byref(x), ctypes.byref(w), ctypes.byref(w), ctypes.byref(bg),
                              None, ctypes.byref(y), 0, None)
    assert rc == nat.EINVAL and "both biases" in nat.last_error()


def test_python_api_refuses_host_tensors(cea):
    q = torch.zeros(1, 2, 2, 8, dtype=torch.bfloat16)
    p = torch.arange(2).view(1, 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cea.attention_with_lse(q, q, q, p, p)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cea.rmsnorm(q.view(4, 8), torch.ones(8, dtype=torch.bfloat16), 1e-5)


def test_python_api_validates_heads_before_device_work(cea):
    q = torch.zeros(1, 2, 4, 8)
    k = torch.zeros(1, 2, 3, 8)
    with pytest.raises(ValueError, match="cannot share"):
        cea.expand_kv(k, 4)
    assert cea.gqa_group(8, 2) == 4
    assert cea.gqa_group(8, 2, [0, 0, 0, 0, 1, 1, 1, 1]) == 4
    assert cea.gqa_group(8, 2, [0, 1, 0, 1, 0, 1, 0, 1]) is None
    with pytest.raises(ValueError, match="one entry per query head"):
        cea.expand_kv(k, 4, kv_map=[0, 1])


OPS = ["attention", "attention_into", "merge", "partitioned", "pack_partial", "merge_packed",
       "ulysses_scatter", "ulysses_gather", "rmsnorm", "rope_tables", "apply_rotary",
       "rmsnorm_rope", "gated_mul", "kv_append", "linear", "linear_into", "linear_gated"]


def test_torch_operator_library_registers_every_op(cea):
    """The PyTorch operator layer (csrc/torch_ops.cpp) loads on top of the C ABI library and
    registers the operators the package dispatches through."""
    assert cea._native.OPS_PATH.exists(), "build the libraries first (__graft_entry__.build())"
    ops = cea._native.ops()
    for name in OPS:
        assert hasattr(ops, name), f"torch.ops.collab_edge.{name} missing"
    # the package's functions go through these operators, not through ctypes
    import inspect

    for mod in (cea.attention, cea.layers, cea.sequence_parallel, cea.kv_cache, cea.projection):
        src = inspect.getsource(mod)
        assert "nat.ops()" in src and "byref" not in src, mod.__name__


def test_operators_refuse_host_tensors(cea):
    """No host path: CPU tensors raise RuntimeError before any work."""
    ops = cea._native.ops()
    q = torch.zeros(1, 4, 2, 8)
    pos = torch.arange(4).view(1, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention(q, q, q, pos, pos, True, 0.35, None, True)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.gated_mul(q.view(4, 16), q.view(4, 16), 0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.linear(q.view(4, 16), q.view(4, 16), None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cea.projection.linear_gated(q.view(4, 16), q.view(4, 16), q.view(4, 16))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cea.attention_with_lse(q, q, q, pos, pos)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cea.rmsnorm(q, torch.ones(8), 1e-5)


def test_missing_libraries_fail_loudly(cea, monkeypatch, tmp_path):
    """No fallback: without the built kernel or operator library every entry raises, naming
    the missing file and how to build it."""
    nat = cea._native
    with pytest.raises(RuntimeError, match="missing: build it"):
        nat.load_library(tmp_path / "libcollab_edge_attn.so")
    monkeypatch.setattr(nat, "_ops", None)
    monkeypatch.setattr(nat, "OPS_PATH", tmp_path / "libcollab_edge_torch.so")
    with pytest.raises(RuntimeError, match="missing: build it"):
        nat.ops()


def test_workspace_counts_decode_partials_only_for_the_decode_route(cea):
    """cea_attention_workspace_bytes adds the split-KV decode partials only for calls the
    decode kernels take (bf16 / f16, head size 64 or 128): f32 and f64 calls of a decode shape
    need the tile summaries alone, so the no-allocation entry point does not refuse them."""
    nat = cea._native
    lib = nat.load_library()
    B, Hq, Sk, Hkv, D = 64, 32, 32768, 8, 128
    tiles = B * ((Sk + 63) // 64) * 32
    bf16 = lib.cea_attention_workspace_bytes(B, 1, Hq, Sk, Hkv, D, 1)
    f32 = lib.cea_attention_workspace_bytes(B, 1, Hq, Sk, Hkv, D, 0)
    f64 = lib.cea_attention_workspace_bytes(B, 1, Hq, Sk, Hkv, D, 3)
    odd = lib.cea_attention_workspace_bytes(B, 1, Hq, Sk, Hkv, 96, 1)
    assert bf16 > (32 << 20) > f32
    assert f32 == f64 == odd == tiles
    # head size 64 takes the decode route as well
    assert lib.cea_attention_workspace_bytes(B, 1, Hq, Sk, Hkv, 64, 1) > tiles


def _split_plan(B, Sq, Hq, Sk, G):
    """Key splits of a bf16 prefill launch, restated from the rule the library documents:
    query heads per workgroup hp in {1, 2, 4, 8} (dividing G) with the fewest padded rows of
    256 / hp per head, one on ties; splits only when the workgroups number fewer than 256,
    then min(16, ceil(512 / workgroups), tiles // 8), at least 2."""
    hp, best = 1, -(-Sq // 256) * 256 - Sq
    for cand in (2, 4, 8):
        if G % cand:
            break
        rows = 256 // cand
        pad = -(-Sq // rows) * rows - Sq
        if pad < best:
            hp, best = cand, pad
    grid = -(-Sq // (256 // hp)) * (Hq // hp) * B
    if grid >= 256:
        return 1
    s = min(16, -(-512 // grid), -(-Sk // 64) // 8)
    return s if s >= 2 else 1


@pytest.mark.parametrize("B,Sq,Hq,Sk,Hkv,D", [
    (1, 128, 32, 32768, 8, 128),   # a prefill chunk: two heads per workgroup, 16 splits
    (1, 300, 8, 3000, 1, 64),      # G = 8
    (4, 128, 32, 32768, 8, 128),   # 64 workgroups: 8 splits
    (1, 8192, 32, 32768, 8, 128),  # the ring share's query block: no split
    (1, 40, 8, 500, 2, 128),       # too few tiles to split
    (2, 33, 6, 4000, 3, 64),       # G = 2
])
def test_workspace_holds_the_key_split_partials(cea, B, Sq, Hq, Sk, Hkv, D):
    """For calls on the prefill route, cea_attention_workspace_bytes is the tile summaries
    (32 bytes per 64-key tile and batch row, rounded up to 256) plus one f32 (out, lse) pair
    per key split."""
    lib = cea._native.load_library()
    tiles = -(-B * -(-Sk // 64) * 32 // 256) * 256
    S = _split_plan(B, Sq, Hq, Sk, Hq // Hkv)
    partials = S * (B * Sq * Hq * D + B * Hq * Sq) * 4 if S > 1 else 0
    assert lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, 1) == tiles + partials
    # f32 calls run other kernels: the summaries alone
    assert lib.cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, 0) == tiles


def _desc(nat, shape, dtype_code, addr):
    """A contiguous cea_tensor over a fake (aligned, never dereferenced) device address."""
    t = nat.CeaTensor()
    t.data = addr
    t.dtype = dtype_code
    t.ndim = len(shape)
    stride = 1
    for i in reversed(range(len(shape))):
        t.size[i] = shape[i]
        t.stride[i] = stride
        stride *= shape[i]
    return t


@pytest.mark.parametrize("B,sizes", [(1, [8192, 8192, 8192, 8192]), (3, [100, 65, 0, 300])])
def test_ring_workspace_covers_every_tile_summary(cea, B, sizes):
    """cea_ring_attention_workspace_bytes for the one-launch route: one 32-byte summary per
    64-key tile of every block and batch row (a workspace sized for the tile count read as a
    key count let the summary pass write past the buffer)."""
    nat = cea._native
    lib = nat.load_library()
    Sq, Hq, Hkv, D = 512, 8, 2, 128
    addr = iter(range(1 << 30, 1 << 40, 1 << 30))
    q = _desc(nat, (B, Sq, Hq, D), 1, next(addr))
    qp = _desc(nat, (B, Sq), 4, next(addr))
    out = _desc(nat, (B, Sq, Hq, D), 1, next(addr))
    n = len(sizes)
    ks = (nat.CeaTensor * n)(*[_desc(nat, (B, s, Hkv, D), 1, next(addr)) for s in sizes])
    vs = (nat.CeaTensor * n)(*[_desc(nat, (B, s, Hkv, D), 1, next(addr)) for s in sizes])
    ps = (nat.CeaTensor * n)(*[_desc(nat, (B, s), 4, next(addr)) for s in sizes])
    got = lib.cea_ring_attention_workspace_bytes(ctypes.byref(q), n, ks, vs, ctypes.byref(qp), ps, 1,
                                                 None, 0, ctypes.byref(out), None)
    tiles = sum((s + 63) // 64 for s in sizes)
    assert got >= B * tiles * 32, (got, B * tiles * 32)
