"""Benchmark of the attention / LSE / layer-op path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input.  The headline workload
is one rank's share of ring-attention prefill (sp=4 zigzag over 32768 tokens, GQA 32/8,
D=128, bf16): 8192 local queries against four 8192-token KV blocks streamed in ring order,
each block merged exactly into the running (out, lse) in the kernel epilogue, output cast to
bf16 (``ring_attention``).  Value = algorithmic TFLOP/s over visible (query, key) pairs.

The same JSON line also reports the other workloads of the path (distributed-KV decode +
merge, RMSNorm+rotary and SiLU-gate, the Ulysses share, the f32 split-merge check), the
roofline of the dominant kernel measured live with HIP events on the launch stream, and the
CPU oracle timed on a bounded sample of the headline workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only ring]
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _measured_traffic(name: str):
    """HBM bytes per launch of a kernel, from the FETCH_SIZE / WRITE_SIZE counter runs
    summarised in profiles/<name>_pmc.md (line ``traffic_bytes_per_launch: N``), or None."""
    path = ROOT / "profiles" / f"{name}_pmc.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def _timed(fn, steps: int, warmup: int, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _graph_timed(fn, steps: int, warmup: int, torch, per_graph: int = 20):
    """Seconds per call of ``fn`` from replays of a HIP graph holding ``per_graph`` calls:
    the GPU time of a launch, without the host's per-call launch cost (which exceeds the
    kernel time of the small layer ops); the median of 5 timed runs."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    for _ in range(max(50, warmup)):  # ~10 ms of back-to-back work: clocks settle
        g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(5):  # median of 5 timed runs of `steps` replays each
        a.record()
        for _ in range(steps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) * 1e-3 / (steps * per_graph))
    return sorted(times)[2]


def bench_ring(cea, torch, steps, warmup, dev):
    w = cea.workloads.ring_share(device=dev)
    comm = cea.LocalGroup(w.layout.num_ranks, w.rank)
    for r, (k, v, p) in enumerate(w.blocks):
        comm.set_shard(r, k=k, v=v, pos=p)
    k0, v0, p0 = w.blocks[w.rank]

    def step():
        return cea.ring_attention(w.q, k0, v0, w.q_pos, p0, comm, w.kv_sizes)

    sec = _timed(step, steps, warmup, torch)
    # average duration of one attention call (tile summary + prefill kernel) over back-to-back
    # ring passes, from two HIP events on the stream the kernels run on (an event pair around
    # every launch would add its own gap and cache flush to each launch)
    stream = torch.cuda.current_stream(dev)
    out = torch.zeros(w.q.shape, dtype=torch.float32, device=dev)
    lse = torch.full((1, w.q.shape[2], w.q.shape[1]), float("-inf"), device=dev)

    def ring_pass():
        for i, src in enumerate(w.ring_order):
            k, v, p = w.blocks[src]
            cea.attention_with_lse_into(out, lse, w.q, k, v, w.q_pos, p, accumulate=i > 0)

    passes = max(3, steps // 2)
    ring_pass()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(passes):
        ring_pass()
    b.record(stream)
    torch.cuda.synchronize()
    launch_ms = a.elapsed_time(b) / (passes * len(w.ring_order))
    flop_launch = w.flop / len(w.ring_order)
    achieved = flop_launch / (launch_ms * 1e-3) / 1e12
    tflops = w.flop / sec / 1e12
    return w, sec, tflops, {
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "traffic": _measured_traffic("attn_prefill_ring_share"),
        "kernel": "attn_prefill_kernel<bf16,128> (+ tile summary pass), one ring step",
        "launch_ms": round(launch_ms, 4),
        "flop_per_launch": int(flop_launch),
    }


def bench_decode(cea, torch, steps, warmup, dev):
    w = cea.workloads.kv_decode(device=dev)
    parts = w.partitions()
    comm = cea.LocalGroup(len(parts), 0)
    for r, (k, v, p) in enumerate(parts):
        comm.set_shard(r, k=k, v=v, pos=p)
    k0, v0, p0 = parts[0]

    def step():
        return cea.distributed_kv_attention(w.q, k0, v0, w.q_pos, p0, comm)

    sec = _timed(step, steps, warmup, torch)
    gbs = w.bytes / sec / 1e9
    return {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
            "ms_per_step": round(sec * 1e3, 4), "bytes": w.bytes,
            "workload": "distributed-KV decode B=32 1 token 32/8 heads D=128 bf16, cache 32768, "
                        "lengths U[1024,32768], 4 partitions 0.4/0.3/0.2/0.1 + exact merge"}


def bench_layers(cea, torch, steps, warmup, dev):
    w = cea.workloads.layer_ops(device=dev)
    inv = cea.layers.rope_inv_freq(w.head_dim, w.theta).to(dev)
    res = {}
    sec = _graph_timed(lambda: cea.rmsnorm_rope(w.x, w.weight, w.eps, w.positions, inv, w.heads),
                       steps, warmup, torch)
    gbs = w.rmsnorm_rope_bytes / sec / 1e9
    res["rmsnorm_rope"] = {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                           "us_per_step": round(sec * 1e6, 2), "bytes": w.rmsnorm_rope_bytes}
    g, u = w.gate, w.up
    sec = _graph_timed(lambda: cea.silu_mul(g, u), steps, warmup, torch)
    gbs = w.silu_bytes / sec / 1e9
    res["silu_mul"] = {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                       "us_per_step": round(sec * 1e6, 2), "bytes": w.silu_bytes}
    res["workload"] = ("bf16 RMSNorm+rotary [4096,4096]->32x128 theta 1e4; SiLU-gate [4096,14336]; "
                       "timed as HIP-graph replays of 20 launches")
    return res


def bench_kv_append(cea, torch, steps, warmup, dev):
    w = cea.workloads.kv_append(device=dev)
    sec = _graph_timed(lambda: cea.kv_append(w.cache_k, w.cache_v, w.cache_pos, w.offset, w.k, w.v,
                                             w.pos, w.cos, w.sin), steps, warmup, torch)
    gbs = w.bytes / sec / 1e9
    return {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
            "us_per_step": round(sec * 1e6, 2), "bytes": w.bytes,
            "workload": "rotary-K + head-major KV-cache append: 8192 tokens x 8 KV heads x 128, "
                        "bf16, into a cache holding 8192 tokens; timed as HIP-graph replays"}


def bench_wire(cea, torch, steps, warmup, dev):
    """The collectives' wire formats on one device: the two Ulysses all-to-alls of rank 0 at
    the Ulysses workload's shape (65536 tokens, 64/16 heads over sp=8, D=128, bf16), and the
    distributed-KV decode workload through the packed all-gather route with the in-place
    merge of the gathered [4, 32, 1, 32, 129] f32 buffer."""
    S, world, D = 65536, 8, 128
    heads = cea.partition_heads(64, 16, world)
    layout = cea.SequenceLayout(S, world, None, "contiguous")
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, S, 64, D, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(1, S, 16, D, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(1, S, 16, D, generator=g, device=dev, dtype=torch.bfloat16)
    pos = torch.arange(S, device=dev).view(1, S)
    grp = cea.LocalGroup(world, 0)
    shards = [tuple(layout.shard(t, r) for t in (q, k, v, pos)) for r in range(world)]
    for r, (a, b, c, p) in enumerate(shards):
        grp.set_shard(r, q=a, k=b, v=c, pos=p)
    me = heads[0]
    width = me.q_count + 2 * me.kv_count
    res = {}
    sec = _graph_timed(lambda: cea.ulysses_scatter(*shards[0], grp, layout.sizes, heads), steps,
                       warmup, torch, per_graph=10)
    nb = 2 * S * width * D * 2 + 2 * S * 8
    res["ulysses_scatter"] = {"value": round(nb / sec / 1e9, 1), "unit": "GB/s",
                              "frac": round(nb / sec / 1e9 / PEAK_HBM_GBS, 4),
                              "us_per_step": round(sec * 1e6, 2), "bytes": nb}
    outs = [torch.randn(1, S, h.q_count, D, generator=g, device=dev, dtype=torch.bfloat16)
            for h in heads]
    sec = _graph_timed(lambda: cea.ulysses_gather(outs, grp, layout.sizes, heads), steps, warmup,
                       torch, per_graph=10)
    nb = 2 * (S // world) * 64 * D * 2
    res["ulysses_gather"] = {"value": round(nb / sec / 1e9, 1), "unit": "GB/s",
                             "frac": round(nb / sec / 1e9 / PEAK_HBM_GBS, 4),
                             "us_per_step": round(sec * 1e6, 2), "bytes": nb}
    del q, k, v, outs, shards, grp
    w = cea.workloads.kv_decode(device=dev)
    parts = w.partitions()
    comm = cea.LocalGroup(len(parts), 0)
    for r, (kk, vv, pp) in enumerate(parts):
        comm.set_shard(r, k=kk, v=vv, pos=pp)
    sec = _timed(lambda: cea.distributed_kv_attention(w.q, *parts[0][:2], w.q_pos, parts[0][2],
                                                      comm, wire=True), steps, warmup, torch)
    B, Sq, Hq, _ = w.q.shape
    gathered = torch.randn(len(parts), B, Sq, Hq, D + 1, device=dev)
    msec = _graph_timed(lambda: cea.merge_packed(gathered, out_dtype=torch.bfloat16), steps,
                        warmup, torch)
    nb = gathered.numel() * 4 + B * Sq * Hq * D * 2
    res["kv_decode_packed"] = {"ms_per_step": round(sec * 1e3, 4),
                               "merge_packed_us": round(msec * 1e6, 2), "merge_bytes": nb,
                               "merge_gbs": round(nb / msec / 1e9, 1)}
    res["workload"] = ("Ulysses sp=8 all-to-alls of rank 0 (65536 tokens, 64/16 heads, D=128, "
                       "bf16; HIP-graph replays); distributed-KV decode via pack + gathered "
                       "[4,32,1,32,129] f32 buffer + in-place merge to bf16")
    return res


def bench_ulysses(cea, torch, steps, warmup, dev):
    w = cea.workloads.ulysses_share(device=dev)

    def step():
        return cea.attention_with_lse(w.q, w.k, w.v, w.pos, w.pos, kv_map=w.kv_map)

    sec = _timed(step, steps, warmup, torch)
    tf = w.flop / sec / 1e12
    return {"value": round(tf, 1), "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
            "ms_per_step": round(sec * 1e3, 4), "flop": w.flop, "valid_tokens": w.valid,
            "workload": "Ulysses sp=8 share: 65536 tokens, 8/2 heads, D=128, bf16, causal, "
                        "4 packed sequences + right padding, emits f32 lse"}


def bench_f32_split(cea, torch, steps, warmup, dev):
    w = cea.workloads.attn_f32_split(device=dev)
    h = w.split

    def step():
        a = cea.attention_with_lse(w.q, w.k[:, :h], w.v[:, :h], w.pos, w.pos[:, :h], scale=w.scale)
        b = cea.attention_with_lse(w.q, w.k[:, h:], w.v[:, h:], w.pos, w.pos[:, h:], scale=w.scale)
        return cea.merge_attention(a[0], a[1], b[0], b[1])

    sec = _timed(step, steps, warmup, torch)
    return {"value": round(w.flop / sec / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(sec * 1e3, 4),
            "workload": "f32 attention B=1 8/8 heads S=512 D=64 causal, 2-way KV split + merge"}


def cpu_baseline(cea, torch, budget_s: float = 20.0):
    """The CPU oracle (restatement of the reference's CPU route) on a bounded sample of the
    headline workload: growing sets of query rows from both zigzag halves, against all four
    KV blocks in ring order, until about ``budget_s`` seconds of CPU work."""
    from oracle import sp_ref

    w = cea.workloads.ring_share(device="cpu")
    # the host share of one GPU: OMP_NUM_THREADS where set, else at most 16 cores
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    half = w.q.shape[1] // 2
    rows, done_s, done_flop, sample = 64, 0.0, 0, []
    while done_s < budget_s and rows <= half:
        idx = torch.cat([torch.arange(0, rows), torch.arange(half, half + rows)])
        q = w.q[:, idx]
        qp = w.q_pos[:, idx]
        t0 = time.perf_counter()
        sp_ref.ring_share(q, qp, w.blocks, w.rank)
        dt = time.perf_counter() - t0
        pairs = sum(cea.workloads.visible_pairs(qp, w.blocks[r][2]) for r in w.ring_order)
        done_s += dt
        done_flop += 4 * w.q.shape[-1] * w.q.shape[2] * pairs
        sample.append(2 * rows)
        rows *= 2
    return {"value": round(done_flop / done_s / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle ring share (CPU flash route, f32) for query-row subsets {sample} "
                      f"of the 8192 local rows (half from each zigzag half) x 4 KV blocks; "
                      f"{done_s:.1f} s, {done_flop:.3e} algorithmic FLOP"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="", help="comma list of: ring,decode,layers,kvappend,ulysses,wire,f32")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="only run a device copy of MIB MiB (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.calib_copy:
        import torch

        n = args.calib_copy * (1 << 20) // 4
        src = torch.randn(n, device="cuda:0")
        dst = torch.empty_like(src)
        sec = _timed(lambda: dst.copy_(src), 10, 2, torch)
        print(json.dumps({"calib_copy_mib": args.calib_copy, "read_bytes": n * 4, "write_bytes": n * 4,
                          "gbs": round(2 * n * 4 / sec / 1e9, 1)}), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build simulates every rank's share on a single "
              "MI355X and has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    import torch

    cea = importlib.import_module("collaborative-edge-system_amd")
    dev = torch.device("cuda:0")
    only = set(filter(None, args.only.split(",")))
    want = lambda name: not only or name in only  # noqa: E731

    w = sec = tflops = roof = None
    if want("ring"):
        _log("ring share (headline)")
        w, sec, tflops, roof = bench_ring(cea, torch, args.steps, args.warmup, dev)
    secondary = {}
    if want("decode"):
        _log("distributed-KV decode")
        secondary["kv_decode"] = bench_decode(cea, torch, args.steps, args.warmup, dev)
    if want("layers"):
        _log("layer ops")
        secondary["layer_ops"] = bench_layers(cea, torch, args.steps, args.warmup, dev)
    if want("kvappend"):
        _log("kv-cache append")
        secondary["kv_append"] = bench_kv_append(cea, torch, args.steps, args.warmup, dev)
    if want("ulysses"):
        _log("ulysses share")
        secondary["ulysses_share"] = bench_ulysses(cea, torch, max(5, args.steps // 2), args.warmup, dev)
    if want("wire"):
        _log("wire formats (Ulysses all-to-alls, packed distributed-KV merge)")
        secondary["wire"] = bench_wire(cea, torch, args.steps, args.warmup, dev)
    if want("f32"):
        secondary["attn_f32_split"] = bench_f32_split(cea, torch, args.steps, args.warmup, dev)
    cpu = None
    if not args.no_cpu_baseline:
        _log("cpu baseline (oracle)")
        cpu = cpu_baseline(cea, torch, args.cpu_budget)

    result = {
        "metric": "attn prefill TFLOP/s (% MFMA peak); decode+merge GB/s (% HBM peak)",
        "value": round(tflops, 2) if w else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4) if w else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1))",
        "config": {
            "workload": "ring_attention share: rank 0 of sp=4 zigzag, 32768 tokens, GQA 32/8, "
                        "D=128, bf16, q 8192 x 4 KV blocks of 8192, online f32 merge",
            "frac_of_peak": round(tflops / PEAK_BF16_TFLOPS, 4) if w else None,
            "flop_per_step": w.flop if w else None,
            "visible_pairs_per_step": w.pairs_per_step if w else None,
            "parallelism": "single GPU, simulated ring (no collectives)",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
