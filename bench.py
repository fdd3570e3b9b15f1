"""Benchmark of the attention / LSE / layer-op path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input.  The headline workload
is one rank's share of ring-attention prefill (sp=4 zigzag over 32768 tokens, GQA 32/8,
D=128, bf16): 8192 local queries against four 8192-token KV blocks streamed in ring order,
each block merged exactly into the running (out, lse) in the kernel epilogue, output cast to
bf16 (``ring_attention``).  Value = algorithmic TFLOP/s over visible (query, key) pairs.

The same JSON line also reports the other workloads of the path (distributed-KV decode +
merge, RMSNorm+rotary and SiLU-gate, the Ulysses share, the f32 split-merge check, the fused
gate/up and Q/K/V projections), the
roofline of the dominant kernel measured live with HIP events on the launch stream, and the
CPU oracle timed on a bounded sample of the headline workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only ring]
       python bench.py --trace-summary <rocprofv3 kernel_trace.csv> [--last N]
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
    """HBM bytes per launch of a kernel, from the TCC request-counter runs summarised in
    profiles/<name>_pmc.md (line ``traffic_bytes_per_launch: N ...``), or None."""
    path = ROOT / "profiles" / f"{name}_pmc.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].split()[0])
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


def _event_timed(fn, steps: int, warmup: int, torch, dev):
    """(wall seconds per call, GPU milliseconds per call from two HIP events on the launch
    stream around the same timed calls)."""
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps, a.elapsed_time(b) / steps


def _event_timed_rounds(fn, steps: int, warmup: int, torch, dev, rounds: int = 5,
                        warm_ms: float = 100.0):
    """For steps of a fraction of a millisecond: warm up for at least ``warm_ms`` of GPU work
    (the clocks settle; a single round right after a few warm-up steps reads several percent
    slow), then ``rounds`` rounds of ``steps`` timed with HIP events.  Returns (wall seconds
    per call of the median round, GPU milliseconds per call of the median round)."""
    _, first_ms = _event_timed(fn, max(1, steps), warmup, torch, dev)
    extra = int(warm_ms / max(first_ms, 1e-3))
    for _ in range(min(extra, 5000)):
        fn()
    res = sorted((_event_timed(fn, steps, 0, torch, dev) for _ in range(rounds)), key=lambda r: r[1])
    return res[len(res) // 2]


def bench_ring(cea, torch, steps, warmup, dev):
    """The headline: ``ring_attention`` over the four KV blocks of the ring share, one
    ``cea_ring_attention`` call (one tile-summary launch over the four blocks + one prefill
    launch that streams them in ring order).  The K timed steps are bracketed by host
    synchronisation (wall clock, ``value``) and by two HIP events on the stream the kernels
    run on; the events give the GPU time of exactly those steps, from which ``roofline``
    takes the average duration of one share's launch pair."""
    w = cea.workloads.ring_share(device=dev)
    comm = cea.LocalGroup(w.layout.num_ranks, w.rank)
    for r, (k, v, p) in enumerate(w.blocks):
        comm.set_shard(r, k=k, v=v, pos=p)
    k0, v0, p0 = w.blocks[w.rank]

    def step():
        return cea.ring_attention(w.q, k0, v0, w.q_pos, p0, comm, w.kv_sizes)

    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    n_launch = 1  # the whole share is one prefill launch
    launch_ms = a.elapsed_time(b) / (steps * n_launch)
    flop_launch = w.flop / n_launch
    achieved = flop_launch / (launch_ms * 1e-3) / 1e12
    tflops = w.flop / sec / 1e12
    return w, sec, tflops, {
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "traffic": _measured_traffic("attn_prefill_ring_share"),
        "kernel": "attn_prefill_kernel<bf16,128> over the 4 KV blocks in ring order (+ tile summary pass), one share",
        "launch_ms": round(launch_ms, 4),
        "launches": steps * n_launch,
        "flop_per_launch": int(flop_launch),
    }


def bench_decode(cea, torch, steps, warmup, dev, hq=32, hkv=8, d=128):
    w = cea.workloads.kv_decode(device=dev, hq=hq, hkv=hkv, d=d)
    parts = w.partitions()
    comm = cea.LocalGroup(len(parts), 0)
    for r, (k, v, p) in enumerate(parts):
        comm.set_shard(r, k=k, v=v, pos=p)
    k0, v0, p0 = parts[0]

    def step():
        return cea.distributed_kv_attention(w.q, k0, v0, w.q_pos, p0, comm)

    # GPU time of the timed steps (HIP events on the launch stream): the step is three short
    # kernels, so the wall clock of 20 steps also holds the host's first-launch latency; the
    # median of 5 rounds after a 100 ms warm-up (steady clocks)
    sec, gpu_ms = _event_timed_rounds(step, steps, warmup, torch, dev)
    gbs = w.bytes / (gpu_ms * 1e-3) / 1e9
    return {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
            "ms_per_step": round(gpu_ms, 4), "wall_ms_per_step": round(sec * 1e3, 4),
            "bytes": w.bytes,
            "workload": f"distributed-KV decode B=32 1 token {hq}/{hkv} heads D={d} bf16, cache 32768, "
                        "lengths U[1024,32768], 4 partitions 0.4/0.3/0.2/0.1 + exact merge"}


def bench_layers(cea, torch, steps, warmup, dev):
    w = cea.workloads.layer_ops(device=dev)
    inv = cea.layers.rope_inv_freq(w.head_dim, w.theta).to(dev)
    res = {}
    rope = lambda: cea.rmsnorm_rope(w.x, w.weight, w.eps, w.positions, inv, w.heads)
    sec = _graph_timed(rope, steps, warmup, torch)
    gbs = w.rmsnorm_rope_bytes / sec / 1e9
    # beside the graph replays: the GPU time per call of direct calls through the operator
    # library, back to back (host dispatch included wherever it exceeds the kernel)
    _, direct_ms = _event_timed(rope, steps, warmup, torch, dev)
    res["rmsnorm_rope"] = {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                           "us_per_step": round(sec * 1e6, 2), "direct_us_per_call": round(direct_ms * 1e3, 2),
                           "bytes": w.rmsnorm_rope_bytes}
    g, u = w.gate, w.up
    silu = lambda: cea.silu_mul(g, u)
    sec = _graph_timed(silu, steps, warmup, torch)
    gbs = w.silu_bytes / sec / 1e9
    _, direct_ms = _event_timed(silu, steps, warmup, torch, dev)
    res["silu_mul"] = {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                       "us_per_step": round(sec * 1e6, 2), "direct_us_per_call": round(direct_ms * 1e3, 2),
                       "bytes": w.silu_bytes}
    for act in ("gelu", "gelu_pytorch_tanh"):  # the reference's other gated activations
        sec = _graph_timed(lambda: cea.gated_mul(g, u, act), steps, warmup, torch)
        gbs = w.silu_bytes / sec / 1e9
        res[f"{act}_mul"] = {"value": round(gbs, 1), "unit": "GB/s",
                             "frac": round(gbs / PEAK_HBM_GBS, 4),
                             "us_per_step": round(sec * 1e6, 2), "bytes": w.silu_bytes}
    res["workload"] = ("bf16 RMSNorm+rotary [4096,4096]->32x128 theta 1e4; SiLU-gate (and the GELU "
                       "gates) [4096,14336]; timed as HIP-graph replays of 20 launches")
    return res


def bench_kv_append(cea, torch, steps, warmup, dev):
    w = cea.workloads.kv_append(device=dev)
    sec = _graph_timed(lambda: cea.kv_append(w.cache_k, w.cache_v, w.cache_pos, w.offset, w.k, w.v,
                                             w.pos, w.cos, w.sin), steps, warmup, torch)
    gbs = w.bytes / sec / 1e9
    _, direct_ms = _event_timed(lambda: cea.kv_append(w.cache_k, w.cache_v, w.cache_pos, w.offset, w.k,
                                                      w.v, w.pos, w.cos, w.sin), steps, warmup, torch, dev)
    return {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
            "us_per_step": round(sec * 1e6, 2), "direct_us_per_call": round(direct_ms * 1e3, 2),
            "bytes": w.bytes,
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
    for j, o in enumerate(outs):  # what the other ranks send back
        grp.set_shard(j, out_heads=o)
    sec = _graph_timed(lambda: cea.ulysses_gather(outs[0], grp, layout.sizes, heads), steps,
                       warmup, torch, per_graph=10)
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
    sec = _timed(lambda: cea.distributed_kv_attention_packed(w.q, *parts[0][:2], w.q_pos,
                                                             parts[0][2], comm), steps, warmup, torch)
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

    sec, gpu_ms = _event_timed(step, steps, warmup, torch, dev)
    tf = w.flop / sec / 1e12
    return {"value": round(tf, 1), "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
            "ms_per_step": round(sec * 1e3, 4), "gpu_ms_per_step": round(gpu_ms, 4),
            "flop": w.flop, "valid_tokens": w.valid,
            "workload": "Ulysses sp=8 share: 65536 tokens, 8/2 heads, D=128, bf16, causal, "
                        "4 packed sequences + right padding, emits f32 lse"}


def bench_prefill_chunk(cea, torch, steps, warmup, dev):
    """A short query block against a long key block: the key-split route (several workgroup
    groups per query block, partials merged) with two query heads per workgroup."""
    w = cea.workloads.prefill_chunk(device=dev)

    def step():
        return cea.attention_with_lse(w.q, w.k, w.v, w.q_pos, w.k_pos)

    sec, gpu_ms = _event_timed_rounds(step, steps, warmup, torch, dev)
    tf = w.flop / (gpu_ms * 1e-3) / 1e12
    return {"value": round(tf, 1), "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
            "ms_per_step": round(gpu_ms, 4), "wall_ms_per_step": round(sec * 1e3, 4),
            "flop": w.flop,
            "workload": "prefill chunk: 128 tokens at batch 1 against 32768 keys, 32/8 heads, "
                        "D=128, bf16, causal, emits f32 lse"}


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


def _paired_timed(fn_a, fn_b, steps: int, warmup: int, torch, dev, rounds: int = 3):
    """Alternating timings of two routes to the same result (``rounds`` x ``steps`` calls each,
    wall clock around host synchronisation, plus HIP events on the launch stream), so both
    see the same clock and power state; returns the best round of each as (wall s, GPU ms)."""
    best = {}
    for _ in range(rounds):
        for key, fn in (("a", fn_a), ("b", fn_b)):
            sec, gpu_ms = _event_timed(fn, steps, warmup, torch, dev)
            if key not in best or sec < best[key][0]:
                best[key] = (sec, gpu_ms)
    return best["a"], best["b"]


def bench_projection(cea, torch, steps, warmup, dev):
    """The fused projections on this package's gfx950 GEMM: gate/up with the SiLU gate in the
    epilogue (one kernel, no [M, 2I] intermediate) against PyTorch's own route to the same
    result (library GEMM + this package's gate kernel), and the Q/K/V projection against
    PyTorch's library GEMM; each pair timed alternately."""
    w = cea.workloads.projections(device=dev)
    n = w.inter
    wg, wu = w.w_gate_up[:n], w.w_gate_up[n:]
    F = torch.nn.functional
    res = {}
    (sec, gpu_ms), (ref_sec, _) = _paired_timed(
        lambda: cea.linear_gated(w.x_mlp, wg, wu, act="silu"),
        lambda: cea.gated_mul(*F.linear(w.x_mlp, w.w_gate_up).split([n, n], -1), "silu"),
        steps, warmup, torch, dev)
    tf = w.flop_gate_up / sec / 1e12
    res["gate_up_silu"] = {"value": round(tf, 1), "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                           "us_per_step": round(sec * 1e6, 1), "gpu_us_per_step": round(gpu_ms * 1e3, 1),
                           "flop": w.flop_gate_up,
                           "torch_route_us": round(ref_sec * 1e6, 1),
                           "speedup_vs_torch_route": round(ref_sec / sec, 3)}
    (sec, gpu_ms), (ref_sec, _) = _paired_timed(lambda: cea.linear(w.x_attn, w.w_qkv),
                                                lambda: F.linear(w.x_attn, w.w_qkv),
                                                steps, warmup, torch, dev)
    tf = w.flop_qkv / sec / 1e12
    res["qkv"] = {"value": round(tf, 1), "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                  "us_per_step": round(sec * 1e6, 1), "gpu_us_per_step": round(gpu_ms * 1e3, 1),
                  "flop": w.flop_qkv, "torch_route_us": round(ref_sec * 1e6, 1),
                  "speedup_vs_torch_route": round(ref_sec / sec, 3)}
    res["workload"] = ("Llama-3-8B-shaped fused projections, bf16: gate/up 4096 tokens x 4096 -> "
                       "2 x 14336 with SiLU fused (torch route: F.linear + gate kernel); Q/K/V 8192 "
                       "tokens x 4096 -> 6144 (torch route: F.linear); best of 3 alternating rounds")
    return res


def _median_time(fn, reps: int) -> float:
    fn()  # one warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def _host_info(threads: int) -> dict:
    import platform

    model = platform.processor() or ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    import torch

    return {"threads": threads, "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "cpu_model": model, "torch": torch.__version__}


def cpu_baseline(cea, torch):
    """The CPU oracle (the restatement of the reference's CPU route: f32 upcast, additive
    -inf bias per query chunk, torch's CPU flash-attention operator, the reference's merges
    and layer-op sequence) on the five workloads, timed on this host's cores with
    ``time.perf_counter``: one warm-up, then the median of N repetitions (N = 5 for the f32
    split-merge, the layer ops and the decode sample; 1 for the ring share, which runs in
    full; the Ulysses share on a stated subset of query rows; 3 for the projections, on 1024
    tokens of each).  Rates use the same
    algorithmic FLOP / byte counts as the GPU lines.  The top-level fields are the headline
    ring share's."""
    from oracle import attention_ref as ref
    from oracle import layers_ref as lref
    from oracle import sp_ref

    # the process's CPU share: OMP_NUM_THREADS where the host sets it (a host shared by several
    # GPUs may give each its own set of cores), else every core this process may run on
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or avail
    torch.set_num_threads(threads)
    configs = {}

    # f32 attention S=512, 8/8 heads, D=64, causal: KV halves + exact merge
    w1 = cea.workloads.attn_f32_split(device="cpu")
    h = w1.split

    def c1():
        a = ref.attention_with_lse(w1.q, w1.k[:, :h], w1.v[:, :h], w1.pos, w1.pos[:, :h], scale=w1.scale)
        b = ref.attention_with_lse(w1.q, w1.k[:, h:], w1.v[:, h:], w1.pos, w1.pos[:, h:], scale=w1.scale)
        return ref.merge_pair(a[0], a[1], b[0], b[1])

    t = _median_time(c1, 5)
    configs["attn_f32_split"] = {"value": round(w1.flop / t / 1e12, 4), "unit": "TFLOP/s",
                                 "ms_per_step": round(t * 1e3, 3), "reps": 5,
                                 "sample": "full workload (two KV halves + merge)"}

    # bf16 RMSNorm+rotary [4096,4096] -> 32x128 and SiLU-gate [4096,14336]
    w2 = cea.workloads.layer_ops(device="cpu")
    inv = lref.inv_freq(w2.head_dim, w2.theta)
    t = _median_time(lambda: lref.rmsnorm_rope(w2.x, w2.weight, w2.eps, w2.positions, inv, w2.heads), 5)
    layer = {"rmsnorm_rope": {"value": round(w2.rmsnorm_rope_bytes / t / 1e9, 2), "unit": "GB/s",
                              "ms_per_step": round(t * 1e3, 3)}}
    t = _median_time(lambda: lref.silu_gate(w2.gate, w2.up), 5)
    layer["silu_mul"] = {"value": round(w2.silu_bytes / t / 1e9, 2), "unit": "GB/s",
                         "ms_per_step": round(t * 1e3, 3)}
    layer["reps"] = 5
    layer["sample"] = "full workload"
    configs["layer_ops"] = layer
    del w2

    # ring share: all 8192 local rows against the four KV blocks, in full
    w3 = cea.workloads.ring_share(device="cpu")
    t0 = time.perf_counter()
    sp_ref.ring_share(w3.q, w3.q_pos, w3.blocks, w3.rank)
    t3 = time.perf_counter() - t0
    ring = {"value": round(w3.flop / t3 / 1e12, 4), "unit": "TFLOP/s",
            "ms_per_step": round(t3 * 1e3, 1), "reps": 1,
            "sample": "full share: 8192 query rows x 4 KV blocks of 8192 in ring order"}
    configs["ring_share"] = ring
    del w3

    # distributed-KV decode: 8 of the 32 sequences (every 4th), 4 partitions + merge
    rows = list(range(0, 32, 4))
    w4 = cea.workloads.kv_decode(device="cpu", batch=rows)
    parts = w4.partitions()
    t = _median_time(lambda: sp_ref.distributed_kv_share(w4.q, w4.q_pos, parts), 5)
    nb = w4.bytes
    configs["kv_decode"] = {"value": round(nb / t / 1e9, 2), "unit": "GB/s",
                            "ms_per_step": round(t * 1e3, 2), "reps": 5, "bytes": nb,
                            "sample": f"sequences {rows} of the 32 (their valid K/V, partials and "
                                      "output bytes), 4 partitions + exact merge"}
    del w4, parts

    # Ulysses share: 32 chunks of 64 query rows, evenly spaced over the valid tokens, against
    # all 65536 keys (the oracle's query chunk is 64 rows at this key count)
    w5 = cea.workloads.ulysses_share(device="cpu")
    L = w5.valid
    starts = torch.linspace(0, max(0, L - 64), 32).round().to(torch.int64)
    idx = torch.cat([torch.arange(int(s0), int(s0) + 64) for s0 in starts])
    qs, ps = w5.q[:, idx], w5.pos[:, idx]
    t = _median_time(lambda: ref.attention_with_lse(qs, w5.k, w5.v, ps, w5.pos, kv_map=w5.kv_map), 1)
    pairs = cea.workloads.visible_pairs(ps, w5.pos)
    flop = 4 * w5.q.shape[-1] * w5.q.shape[2] * pairs
    configs["ulysses_share"] = {"value": round(flop / t / 1e12, 4), "unit": "TFLOP/s",
                                "seconds": round(t, 3), "reps": 1,
                                "sample": f"{idx.numel()} of {L} valid query rows (32 evenly "
                                          "spaced chunks of 64) x 65536 keys"}
    del w5

    # fused projections: 1024 of the 4096 gate/up tokens (the oracle's F.linear on the CPU in
    # bf16, then act(gate) * up) and 1024 of the 8192 Q/K/V tokens
    w6 = cea.workloads.projections(device="cpu")
    xs, xa = w6.x_mlp[:1024], w6.x_attn[:1024]
    n6 = w6.inter
    t = _median_time(lambda: lref.gated(lref.linear(xs, w6.w_gate_up[:n6]),
                                        lref.linear(xs, w6.w_gate_up[n6:]), "silu"), 3)
    proj = {"gate_up_silu": {"value": round(w6.flop_gate_up * 1024 / w6.x_mlp.shape[0] / t / 1e12, 4),
                             "unit": "TFLOP/s", "ms_per_step": round(t * 1e3, 2)}}
    t = _median_time(lambda: lref.linear(xa, w6.w_qkv), 3)
    proj["qkv"] = {"value": round(w6.flop_qkv * 1024 / w6.x_attn.shape[0] / t / 1e12, 4),
                   "unit": "TFLOP/s", "ms_per_step": round(t * 1e3, 2)}
    proj["reps"] = 3
    proj["sample"] = "1024 tokens of each projection, full weights"
    configs["projection"] = proj
    del w6

    return {"value": ring["value"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": ring["sample"] + "; the other workloads under 'configs'",
            "host": _host_info(threads), "configs": configs}


def summarize_kernel_trace(path: str, last: int) -> str:
    """Per-kernel duration statistics of the last ``last`` dispatches of each kernel in a
    rocprofv3 kernel-trace CSV (``--kernel-trace --output-format csv``): the dispatches of a
    bench run's timed steps, without its warm-up."""
    import csv

    rows = {}
    with open(path, newline="") as f:
        for rec in csv.DictReader(f):
            name = rec.get("Kernel_Name") or rec.get("KernelName") or "?"
            t0 = int(rec.get("Start_Timestamp") or rec.get("BeginNs"))
            t1 = int(rec.get("End_Timestamp") or rec.get("EndNs"))
            rows.setdefault(name, []).append((t0, t1 - t0))
    lines = ["| kernel | dispatches (all) | averaged | avg us | min us | max us |",
             "|---|---|---|---|---|---|"]
    for name, recs in sorted(rows.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        recs.sort()
        tail = [d for _, d in recs[-last:]]
        short = name if len(name) < 90 else name[:87] + "..."
        lines.append(f"| `{short}` | {len(recs)} | {len(tail)} | {sum(tail) / len(tail) / 1e3:.2f} "
                     f"| {min(tail) / 1e3:.2f} | {max(tail) / 1e3:.2f} |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the shader clock settles over the first ~25 ms of back-to-back shares (the first
    # dispatches of a process run up to 30 % slow): 20 warm-up shares (~40 ms) reach it
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of: ring,decode,layers,kvappend,ulysses,chunk,wire,f32,proj")
    ap.add_argument("--trace-summary", default="", metavar="CSV",
                    help="only summarise a rocprofv3 kernel-trace CSV (the last --last "
                         "dispatches of every kernel) and exit")
    ap.add_argument("--last", type=int, default=80)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="only run a device copy of MIB MiB (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.trace_summary:
        print(summarize_kernel_trace(args.trace_summary, args.last))
        return 0
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
        print("bench.py measures one GPU: this package simulates every rank's share on a single "
              "MI355X and has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    import torch

    cea = importlib.import_module("collaborative-edge-system_amd")
    dev = torch.device("cuda:0")
    only = set(filter(None, args.only.split(",")))
    want = lambda name: not only or name in only  # noqa: E731

    # The secondary lines run first (the graph-timed layer ops ahead of the decode, so no
    # event-timed line is a process's first GPU work) and the headline right after them,
    # with no idle gap: a GPU coming out of idle raises its shader clock over the first ~25 ms
    # of back-to-back work (a process's first shares run up to 30 % slow), so W warm-up
    # shares of a few milliseconds would leave part of the timed shares inside that ramp.
    secondary = {}
    if want("layers"):
        _log("layer ops")
        secondary["layer_ops"] = bench_layers(cea, torch, args.steps, args.warmup, dev)
    if want("kvappend"):
        _log("kv-cache append")
        secondary["kv_append"] = bench_kv_append(cea, torch, args.steps, args.warmup, dev)
    if want("decode"):
        _log("distributed-KV decode")
        secondary["kv_decode"] = bench_decode(cea, torch, args.steps, args.warmup, dev)
        # the same step at the tinyllama-1.1b preset's heads (32 query / 4 KV, head size 64)
        secondary["kv_decode_d64"] = bench_decode(cea, torch, args.steps, args.warmup, dev,
                                                  hq=32, hkv=4, d=64)
    if want("ulysses"):
        _log("ulysses share")
        secondary["ulysses_share"] = bench_ulysses(cea, torch, max(5, args.steps // 2), args.warmup, dev)
    if want("chunk"):
        _log("prefill chunk against a long key block")
        secondary["prefill_chunk"] = bench_prefill_chunk(cea, torch, args.steps, args.warmup, dev)
    if want("wire"):
        _log("wire formats (Ulysses all-to-alls, packed distributed-KV merge)")
        secondary["wire"] = bench_wire(cea, torch, args.steps, args.warmup, dev)
    if want("f32"):
        secondary["attn_f32_split"] = bench_f32_split(cea, torch, args.steps, args.warmup, dev)
    if want("proj"):
        _log("fused projections (gate/up + SiLU, Q/K/V)")
        secondary["projection"] = bench_projection(cea, torch, 10, max(5, args.warmup), dev)
    w = sec = tflops = roof = None
    if want("ring"):
        _log("ring share (headline)")
        w, sec, tflops, roof = bench_ring(cea, torch, args.steps, args.warmup, dev)
    cpu = None
    if not args.no_cpu_baseline:
        _log("cpu baseline (oracle)")
        cpu = cpu_baseline(cea, torch)

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
