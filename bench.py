"""Benchmark of the fracture_amd hot path on one MI355X.

Default workload (the metric's configuration): one Llama-3.1-8B decode step's elementwise
chain at batch 64, fp16 — embedding gather from a [128256, 4096] table, RoPE on
Q [64, 32, 128] and K [64, 8, 128] (theta 500000, positions in [0, 8192)), SwiGLU on
[64, 14336], and two residual adds fused with RMSNorm on [64, 4096] — with inputs in device
memory. A step is the five launches; 20 consecutive steps are captured in one HIP graph
(`--steps-per-graph`) and replayed (eager timing reported too). Replaying one set of inputs
keeps its 12 MB in L2 / MALL, as activations written by the previous kernel of a real step
would be; `cold_inputs` repeats the measurement over 40 input sets (more than the 256 MB MALL)
so that every step reads its inputs from HBM.

Printed: one JSON line with the metric (whole-chain algorithmic GB/s; ms_per_step), per-kernel
microseconds and GB/s, the roofline object for the kernel that takes the most time per step,
compact results of the other configurations (`configs`: prefill-shaped reductions, TurboQuant
compress / dequantize, TurboQuant decode attention both over contiguous pools and through the
handle runtime over per-block tensors) and the CPU baseline: the oracle's restatement of the
reference's CPU formulas on this host, one thread and all host cores (up to 16), for the chain
and for every configuration (bounded samples, scaled to the full workload).

Other workloads (parity-tested configurations, printed as their own JSON lines):
  --workload prefill      add+RMSNorm [8192,4096], SwiGLU [8192,14336], softmax/argmax [64,128256]
  --workload tq           TurboQuant compress + dequantize of K and V [32768, 8, 128], 4 and 3 bit
  --workload attention    decode attention over a K4/V4 page pool, B=64, 32/8 heads, ctx U[1024,32768],
                          and causal prefill of one sequence (2048 over 2048, 512 over 8192 positions)
  --workload paged        the same decode attention and prefill over FP16 pages (attention_paged.cu)
  --workload floors       the floors the decode-chain kernels and the [64,128256] reductions are
                          compared with: an empty kernel, and probes that move each kernel's bytes
                          and compute nothing (also part of the default and prefill lines)

HBM traffic (the roofline's "traffic" field, from profiles/traffic.json):
  rocprofv3 --pmc FETCH_SIZE -d <F> -o pmc -- python3 bench.py --workload pmc
  rocprofv3 --pmc WRITE_SIZE -d <W> -o pmc -- python3 bench.py --workload pmc
  python3 bench.py --traffic-from <F> <W>      (writes profiles/traffic.json, prints a table)
The pmc workload runs a 1 GiB device copy (calibration: the counters' reading for a known
number of bytes) and then every operation below once, each after a 4 KiB copy that marks
where its dispatches start.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
METRIC = "HBM GB/s (% of peak) per kernel; µs per B=64 decode-step elementwise chain"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "prefill", "tq", "attention", "paged", "floors", "all",
                             "pmc"])
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc runs of --workload pmc into "
                         "profiles/traffic.json")
    ap.add_argument("--ktrace-from", metavar="TRACE_DIR",
                    help="print a markdown summary of a rocprofv3 --kernel-trace run")
    ap.add_argument("--counters-from", nargs="+", metavar="PMC_DIR",
                    help="print per-kernel averages of rocprofv3 --pmc runs (one dir per pass)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="default run: leave out the other configurations' results")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="time the chain without a HIP graph")
    ap.add_argument("--steps-per-graph", type=int, default=20,
                    help="decode-chain steps captured in one HIP graph (1: one graph per step)")
    return ap.parse_args()


def gbs(nbytes: float, us: float) -> float:
    return nbytes / (us * 1e-6) / 1e9


class Timer:
    """HIP events on torch's current stream, which is the stream the kernels launch on."""

    def __init__(self, torch):
        self.torch = torch

    def time_us(self, fn, reps: int, warmup: int = 3, groups: int = 5,
                warm_ms: float = 30.0) -> float:
        """Median over `groups` timed groups of `reps` back-to-back eager calls (for launches of
        >= ~10 us, where the host keeps the queue full). Warm-up runs at least `warmup` calls
        and at least `warm_ms` of GPU time: the first few milliseconds of a burst run at lower
        shader clocks (a 400 us kernel measured ~20% slower in its first calls)."""
        t = self.torch
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        t.cuda.synchronize()
        s.record()
        n = 0
        while True:
            fn()
            n += 1
            if n >= warmup and n % 4 == 0:
                e.record()
                e.synchronize()
                if s.elapsed_time(e) >= warm_ms or n >= 2000:
                    break
        per = []
        for _ in range(groups):
            s.record()
            for _ in range(reps):
                fn()
            e.record()
            e.synchronize()
            per.append(s.elapsed_time(e) * 1e3 / reps)
        per.sort()
        return per[len(per) // 2]

    def graph_time_us(self, fn, per_graph: int = 50, replays: int = 20) -> float:
        """Average launch duration of `fn` from a HIP graph of `per_graph` back-to-back calls
        replayed `replays` times (short launches, which host-side launch cost would hide)."""
        t = self.torch
        side = t.cuda.Stream()
        side.wait_stream(t.cuda.current_stream())
        with t.cuda.stream(side):
            for _ in range(3):
                fn()
        t.cuda.current_stream().wait_stream(side)
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g):
            for _ in range(per_graph):
                fn()
        g.replay()
        t.cuda.synchronize()
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(replays):
            g.replay()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) * 1e3 / (replays * per_graph)


def traffic_of(kernel_key: str):
    """HBM bytes per dispatch measured with rocprofv3 PMC counters, when recorded."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kernel_key, {}).get("bytes_per_dispatch")
    except (ValueError, OSError):
        return None


# ---------------------------------------------------------------------------------------
# decode-step chain (the headline)
# ---------------------------------------------------------------------------------------
def decode_inputs(torch, dev, seed=0, table=None):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, V, H, QH, KVH, HD, FF = 64, 128256, 4096, 32, 8, 128, 14336
    f16 = torch.float16
    x = {}
    x["table"] = table if table is not None else (
        torch.randn((V, H), generator=g, device=dev) * 0.02).to(f16)
    x["ids"] = torch.randint(0, V, (B,), generator=g, device=dev, dtype=torch.int32)
    x["emb"] = torch.empty((B, H), dtype=f16, device=dev)
    x["q"] = torch.randn((B, QH, HD), generator=g, device=dev).to(f16)
    x["k"] = torch.randn((B, KVH, HD), generator=g, device=dev).to(f16)
    x["pos"] = torch.randint(0, 8192, (B,), generator=g, device=dev, dtype=torch.int32)
    from fracture_amd import turboquant as tq

    x["freqs"] = torch.from_numpy(tq.rope_freqs(HD, 500000.0)).to(dev)
    x["gate"] = torch.randn((B, FF), generator=g, device=dev).to(f16)
    x["up"] = torch.randn((B, FF), generator=g, device=dev).to(f16)
    x["act"] = torch.empty((B, FF), dtype=f16, device=dev)
    x["h"] = torch.randn((B, H), generator=g, device=dev).to(f16)
    x["d1"] = torch.randn((B, H), generator=g, device=dev).to(f16)
    x["d2"] = torch.randn((B, H), generator=g, device=dev).to(f16)
    x["w1"] = (torch.rand((H,), generator=g, device=dev) + 0.5).to(f16)
    x["w2"] = (torch.rand((H,), generator=g, device=dev) + 0.5).to(f16)
    x["n1"] = torch.empty((B, H), dtype=f16, device=dev)
    x["n2"] = torch.empty((B, H), dtype=f16, device=dev)
    return x


def decode_input_sets(torch, dev, n, base):
    """n further sets of the chain's activations (ids, positions, q/k, gate/up, h/deltas and
    outputs), sharing the table, frequencies and norm weights of `base`."""
    sets = []
    for i in range(n):
        x = decode_inputs(torch, dev, seed=100 + i, table=base["table"])
        for k in ("freqs", "w1", "w2"):
            x[k] = base[k]
        sets.append(x)
    return sets


# launches of each kernel per decode step
DECODE_COUNTS = {"embedding": 1, "rope": 1, "silu_mul": 1, "add_rmsnorm": 2}
DECODE_KERNELS = {"embedding": "embedding_vec_kernel", "rope": "rope_wave_kernel<fp16>",
                  "silu_mul": "silu_mul_vec_kernel<fp16>",
                  "add_rmsnorm": "rmsnorm_vec_kernel<fp16, residual, 1>"}


def cpu_threads() -> int:
    """Host threads for the all-core CPU baseline: the cores this process may run on, at most
    16 (one GPU's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def par_rows(fn, arrays, rows, threads):
    """fn(*row_slices) over `threads` contiguous row ranges of `arrays` at once (the oracle's C
    functions release the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    cuts = [rows * i // threads for i in range(threads + 1)]
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda i: fn(*(a[cuts[i]:cuts[i + 1]] for a in arrays)), range(threads)))


def median_time(fn, min_runs=3, seconds=1.0):
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def decode_bytes():
    B, H, QH, KVH, HD, FF = 64, 4096, 32, 8, 128, 14336
    return {
        "embedding": 2 * B * H * 2 + B * 4,
        "rope": 2 * B * (QH + KVH) * HD * 2 + B * 4 + HD // 2 * 4,
        "silu_mul": 3 * B * FF * 2,
        "add_rmsnorm": 4 * B * H * 2 + H * 2,
    }


def decode_ops(K, x):
    return {
        "embedding": lambda: K.embedding(x["emb"], x["table"], x["ids"]),
        "rope": lambda: K.rope(x["q"], x["k"], x["pos"], x["freqs"]),
        "silu_mul": lambda: K.silu_mul(x["act"], x["gate"], x["up"]),
        "add_rmsnorm": lambda: K.add_rmsnorm(x["h"], x["d1"], x["w1"], 1e-5, x["n1"]),
        "add_rmsnorm_2": lambda: K.add_rmsnorm(x["h"], x["d2"], x["w2"], 1e-5, x["n2"]),
    }


def runtime_decode_graph(steps_per_graph: int, replays: int) -> float:
    """µs per step of the decode chain captured through the handle runtime's graph API
    (per_graph consecutive steps per graph, as the raw-launcher timing), with its own tensors
    of the chain's shapes."""
    import numpy as np

    from fracture_amd import DType, HipBackend

    B, V, H, QH, KVH, HD, FF = 64, 128256, 4096, 32, 8, 128, 14336
    rng = np.random.default_rng(1)
    with HipBackend(0) as be:
        be.precompute_rope_freqs(HD, 500000.0)
        f16 = DType.FP16
        # finite fp16 values in [0, 2): bit patterns below 0x4000
        table = be.upload(rng.integers(0, 0x4000, (V, H), dtype=np.uint16).view(np.float16))
        ids = be.alloc([B], DType.FP32)
        be.copy_to_device(ids, rng.integers(0, V, B).astype(np.uint32))
        pos = be.alloc([B], DType.FP32)
        be.copy_to_device(pos, rng.integers(0, 8192, B).astype(np.uint32))
        t = {n: be.upload(rng.standard_normal(shape).astype(np.float16)) for n, shape in
             (("q", (B, QH, HD)), ("k", (B, KVH, HD)), ("gate", (B, FF)), ("up", (B, FF)),
              ("h", (B, H)), ("d1", (B, H)), ("d2", (B, H)))}
        w1 = be.upload(rng.uniform(0.5, 1.5, H).astype(np.float16))
        w2 = be.upload(rng.uniform(0.5, 1.5, H).astype(np.float16))
        emb, act = be.alloc([B, H], f16), be.alloc([B, FF], f16)
        n1, n2 = be.alloc([B, H], f16), be.alloc([B, H], f16)

        def steps():
            for _ in range(steps_per_graph):
                be.embedding_dev(ids, B, table, emb)
                be.rope_dev(t["q"], t["k"], pos, B, HD)
                be.silu_mul(t["gate"], t["up"], act)
                be.add_rmsnorm(t["h"], t["d1"], w1, 1e-5, n1)
                be.add_rmsnorm(t["h"], t["d2"], w2, 1e-5, n2)

        g = be.capture(steps)
        for _ in range(2):
            be.graph_launch(g)
        be.synchronize()
        tm = be.create_timer()
        be.start_timer(tm)
        for _ in range(replays):
            be.graph_launch(g)
        ms = be.stop_timer(tm)
        be.synchronize()
        be.destroy_timer(tm)
        be.graph_destroy(g)
    return ms * 1e3 / (replays * steps_per_graph)


def decode_step(ops):
    for f in ops.values():
        f()


def cpu_decode_baseline(seconds: float, threads: int = 1):
    """The oracle's restatement of the reference's CPU formulas for the same chain, on one
    thread or split by rows over `threads`, median over as many steps as fit in `seconds`
    (at least 3)."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0)
    B, V, H, QH, KVH, HD, FF = 64, 128256, 4096, 32, 8, 128, 14336
    table = (np.arange(V, dtype=np.int64)[:, None] * 2654435761 + np.arange(H)[None, :] * 40503)
    table = (table % 30000).astype(np.int16).view(np.float16)
    ids = rng.integers(0, V, B).astype(np.uint32)
    q = rng.standard_normal((B, QH, HD)).astype(np.float16)
    k = rng.standard_normal((B, KVH, HD)).astype(np.float16)
    pos = rng.integers(0, 8192, B).astype(np.uint32)
    fr = oracle.rope_freqs(HD, 500000.0)
    g = rng.standard_normal((B, FF)).astype(np.float16)
    u = rng.standard_normal((B, FF)).astype(np.float16)
    h = rng.standard_normal((B, H)).astype(np.float16)
    d1 = rng.standard_normal((B, H)).astype(np.float16)
    d2 = rng.standard_normal((B, H)).astype(np.float16)
    w = rng.uniform(0.5, 1.5, H).astype(np.float16)

    def step1(h):
        oracle.embedding(table, ids)
        oracle.rope(q, pos, fr)
        oracle.rope(k, pos, fr)
        oracle.silu_mul(g, u)
        h, _ = oracle.add_rmsnorm(h, d1, w, 1e-5)
        h, _ = oracle.add_rmsnorm(h, d2, w, 1e-5)
        return h

    def step_par(h):
        par_rows(lambda i: oracle.embedding(table, i), [ids], B, threads)
        par_rows(lambda a, p: oracle.rope(a, p, fr), [q, pos], B, threads)
        par_rows(lambda a, p: oracle.rope(a, p, fr), [k, pos], B, threads)
        par_rows(oracle.silu_mul, [g, u], B, threads)
        par_rows(lambda a, b: oracle.add_rmsnorm(a, b, w, 1e-5), [h, d1], B, threads)
        par_rows(lambda a, b: oracle.add_rmsnorm(a, b, w, 1e-5), [h, d2], B, threads)
        return h

    state = {"h": h}

    def run():
        state["h"] = step1(state["h"]) if threads == 1 else step_par(state["h"])

    med, n = median_time(run, 3, seconds)
    return med * 1e6, n


# What each measured kernel moves (inputs read, outputs written, bytes of each), for the probe
# that stands for it: the same traffic with no arithmetic (fhip_probe_stream).
FLOOR_TRAFFIC = {
    "embedding": (1, 1, 64 * 4096 * 2),                 # 64 table rows in, 64 rows out
    "rope": (1, 1, 64 * (32 + 8) * 128 * 2),            # Q and K in place
    "silu_mul": (2, 1, 64 * 14336 * 2),
    "add_rmsnorm": (2, 2, 64 * 4096 * 2),               # h, delta in; h, normed out
    "softmax_64x128256": (1, 1, 64 * 128256 * 4),       # one read, one write
    "argmax_64x128256": (1, 0, 64 * 128256 * 4),        # one read
}
FLOOR_GRIDS = (64, 128, 256, 512, 1024, 2048, 4096, 8192)


def graph_seq_time_us(torch, fns, replays: int = 20) -> float:
    """Average launch duration of the calls `fns` captured in order in one HIP graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns[:3]:
            f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e3 / (replays * len(fns))


def run_floors(torch, K, dev):
    """The floors each kernel is compared with, timed the way the kernels are (a HIP graph of
    50 back-to-back launches, replayed): an empty kernel, and for each kernel a probe that
    moves the same bytes (inputs read, outputs written) and computes nothing, at the best of
    a sweep of grid sizes. `cold` variants cycle over buffers larger in total than the MALL
    (256 MB), so every launch reads from HBM."""
    timer = Timer(torch)
    out = {"empty_kernel_us": {f"grid_{g}": round(timer.graph_time_us(lambda g=g: K.probe_empty(g)), 3)
                               for g in (1, 64, 256, 1024)}}
    sink = torch.empty(256, dtype=torch.int32, device=dev)
    big = 64 * 128256 * 4
    pool = [torch.empty(big // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(5)]

    def probe(nin, nout, nb, bufs=pool):
        best = None
        for g in FLOOR_GRIDS:
            if g > max(1, nb // 16 // 256) * 2:
                break
            us = timer.graph_time_us(lambda g=g: K.probe_stream(bufs[:nin], bufs[nin:nin + nout],
                                                                 nb, g, sink))
            if best is None or us < best[0]:
                best = (us, g)
        return {"us": round(best[0], 3), "grid": best[1], "bytes": nb * (nin + nout),
                "GB/s": round(gbs(nb * (nin + nout), best[0]), 1)}

    for name, (nin, nout, nb) in FLOOR_TRAFFIC.items():
        out[name] = probe(nin, nout, nb)
    for mib in (1, 2, 6):
        out[f"copy_{mib}MiB"] = probe(1, 1, mib << 20)
    # cold: 12 sets of the 32.8 MB logits-sized buffers (394 MB), one per launch
    sets = [torch.empty(big // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(12)]
    grid = out["argmax_64x128256"]["grid"]
    us = graph_seq_time_us(torch, [lambda b=b: K.probe_stream([b], [], big, grid, sink)
                                   for b in sets * 4])
    out["argmax_64x128256_cold"] = {"us": round(us, 3), "grid": grid, "bytes": big,
                                    "GB/s": round(gbs(big, us), 1)}
    outs = [torch.empty_like(sets[0]) for _ in range(12)]
    grid = out["softmax_64x128256"]["grid"]
    us = graph_seq_time_us(torch, [lambda i=i: K.probe_stream([sets[i]], [outs[(i + 5) % 12]],
                                                              big, grid, sink)
                                   for i in range(12)] * 4)
    out["softmax_64x128256_cold"] = {"us": round(us, 3), "grid": grid, "bytes": 2 * big,
                                     "GB/s": round(gbs(2 * big, us), 1)}
    del sets, outs, pool
    torch.cuda.synchronize()
    return out


def with_floor(entry, floor):
    """entry (a kernel's us) beside the floor of its traffic: floor_us / us."""
    entry["floor_us"] = floor["us"]
    entry["frac_of_floor"] = round(floor["us"] / entry["us"], 3)
    return entry


def run_decode(args, torch, K, dev):
    x = decode_inputs(torch, dev)
    ops = decode_ops(K, x)
    nbytes = decode_bytes()
    chain_bytes = (nbytes["embedding"] + nbytes["rope"] + nbytes["silu_mul"] +
                   2 * nbytes["add_rmsnorm"])
    timer = Timer(torch)
    torch.cuda.synchronize()

    # A graph holds `per_graph` consecutive steps, as a serving loop captures a whole decode
    # step (every layer's kernels) in one graph: the per-launch cost of a graph is then shared
    # by many kernels instead of landing on five. The timed region is exactly args.steps
    # steps: full graphs, then one graph of the remaining steps.
    per_graph = max(1, min(args.steps_per_graph, args.steps))
    graphs = {}
    if not args.eager:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                decode_step(ops)  # warm the launch path on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        for n in {per_graph, args.steps % per_graph} - {0}:
            graphs[n] = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graphs[n]):
                for _ in range(n):
                    decode_step(ops)
        torch.cuda.synchronize()

    def run_steps(n):
        if args.eager:
            for _ in range(n):
                decode_step(ops)
            return
        for _ in range(n // per_graph):
            graphs[per_graph].replay()
        if n % per_graph:
            graphs[n % per_graph].replay()

    for _ in range(args.warmup):  # untimed: the warmup steps, then each graph once
        decode_step(ops)
    for g_ in graphs.values():
        g_.replay()
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s_ev.record()
    run_steps(args.steps)
    e_ev.record()
    torch.cuda.synchronize()
    us_step = s_ev.elapsed_time(e_ev) * 1e3 / args.steps
    eager_us = timer.time_us(lambda: decode_step(ops), max(20, args.steps // 4))

    # the same chain with every step on its own inputs (40 sets, ~370 MB: more than the MALL),
    # so that each step reads its activations from HBM
    cold_us = None
    if not args.eager:
        sets = decode_input_sets(torch, dev, 40, x)
        cold_ops = [decode_ops(K, xs) for xs in sets]
        gc = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gc):
            for o in cold_ops:
                decode_step(o)
        gc.replay()
        torch.cuda.synchronize()
        reps = max(1, args.steps // len(cold_ops))
        s_ev.record()
        for _ in range(reps):
            gc.replay()
        e_ev.record()
        torch.cuda.synchronize()
        cold_us = s_ev.elapsed_time(e_ev) * 1e3 / (reps * len(cold_ops))
        del gc, cold_ops, sets

    # per-kernel average launch durations (back-to-back launches between two events)
    per = {}
    for name in ("embedding", "rope", "silu_mul", "add_rmsnorm"):
        us = timer.graph_time_us(ops[name])
        per[name] = {"us": round(us, 3), "GB/s": round(gbs(nbytes[name], us), 1),
                     "frac_of_peak": round(gbs(nbytes[name], us) / PEAK_HBM_GBS, 4),
                     "bytes": nbytes[name],
                     "traffic": traffic_of({"embedding": "decode_embedding", "rope": "decode_rope",
                                            "silu_mul": "silu_mul_64x14336",
                                            "add_rmsnorm": "decode_add_rmsnorm"}[name])}
    floors = run_floors(torch, K, dev)
    for name, e in per.items():
        with_floor(e, floors[name])
    # the roofline kernel: the one that takes the most time per step (launches x duration)
    for name, e in per.items():
        e["launches_per_step"] = DECODE_COUNTS[name]
        e["us_per_step"] = round(e["us"] * DECODE_COUNTS[name], 3)
    dom = max(per, key=lambda n: per[n]["us_per_step"])
    traffic_key = {"embedding": "decode_embedding", "rope": "decode_rope",
                   "silu_mul": "silu_mul_64x14336", "add_rmsnorm": "decode_add_rmsnorm"}[dom]
    roof = {"kernel": DECODE_KERNELS[dom], "bound": "hbm",
            "achieved": per[dom]["GB/s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(per[dom]["GB/s"] / PEAK_HBM_GBS, 4),
            "traffic": traffic_of(traffic_key), "algorithmic_bytes": nbytes[dom],
            "avg_launch_us": per[dom]["us"],
            "launches_per_step": DECODE_COUNTS[dom],
            "floor_us": per[dom]["floor_us"], "frac_of_floor": per[dom]["frac_of_floor"],
            "note": "average launch duration from a HIP graph of 50 back-to-back launches "
                    "(HIP events on the launch stream); floor_us is a kernel that moves the "
                    "same bytes and computes nothing, timed the same way (floors.add_rmsnorm); "
                    "an empty kernel costs floors.empty_kernel_us per launch"}

    result = {
        "metric": METRIC,
        "value": round(gbs(chain_bytes, us_step), 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "us_per_step": round(us_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded torch.Generator; Llama-3.1-8B shapes)",
        "config": {"workload": "llama3.1-8b decode-step elementwise chain, batch 64, fp16",
                   "batch": 64, "hidden": 4096, "vocab": 128256, "q_heads": 32,
                   "kv_heads": 8, "head_dim": 128, "ffn": 14336, "rope_theta": 500000.0,
                   "launch": "eager" if args.eager else f"hip graph, {per_graph} steps per graph",
                   "chain_bytes": chain_bytes},
        "eager_us_per_step": round(eager_us, 3),
        "cold_inputs": None if cold_us is None else {
            "us_per_step": round(cold_us, 3), "GB/s": round(gbs(chain_bytes, cold_us), 1),
            "input_sets": 40},
        "kernels": per,
        "roofline": roof,
        "floors": floors,
    }
    if not args.eager:
        rt_us = runtime_decode_graph(per_graph, max(1, args.steps // per_graph))
        result["handle_runtime_graph"] = {
            "us_per_step": round(rt_us, 3), "GB/s": round(gbs(chain_bytes, rt_us), 1),
            "steps_per_graph": per_graph,
            "note": "the same chain through the handle runtime: fhip_embedding_dev, "
                    "fhip_rope_dev, fhip_silu_mul, 2x fhip_add_rmsnorm captured with "
                    "fhip_graph_begin / fhip_graph_end, replayed with fhip_graph_launch; "
                    "HIP events on the backend stream"}
    if not args.no_cpu_baseline:
        cpu_us, n = cpu_decode_baseline(args.cpu_seconds / 2)
        th = cpu_threads()
        cpu_par, n2 = cpu_decode_baseline(args.cpu_seconds / 2, th)
        result["cpu_baseline"] = {
            "value": round(gbs(chain_bytes, cpu_us), 3), "unit": "GB/s", "cores": 1,
            "kind": "port", "us_per_step": round(cpu_us, 1),
            "sample": f"median of {n} steps of the same chain (same shapes) through the C "
                      f"restatement of the reference's CPU formulas, one thread",
            "all_cores": {"cores": th, "us_per_step": round(cpu_par, 1),
                          "value": round(gbs(chain_bytes, cpu_par), 3),
                          "sample": f"median of {n2} steps, each op split by rows over {th} "
                                    f"threads"},
            "host": host_cpu()}
    return result


def host_cpu():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "threads_used": cpu_threads()}


# ---------------------------------------------------------------------------------------
# other workloads
# ---------------------------------------------------------------------------------------
def run_prefill(args, torch, K, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    f16 = torch.float16
    h = torch.randn((8192, 4096), generator=g, device=dev).to(f16)
    d = torch.randn((8192, 4096), generator=g, device=dev).to(f16)
    w = (torch.rand((4096,), generator=g, device=dev) + 0.5).to(f16)
    n = torch.empty_like(h)
    gate = torch.randn((8192, 14336), generator=g, device=dev).to(f16)
    up = torch.randn((8192, 14336), generator=g, device=dev).to(f16)
    act = torch.empty_like(gate)
    lg = torch.randn((64, 128256), generator=g, device=dev) * 3
    lg[torch.arange(64, device=dev), torch.randint(0, 128256, (64,), generator=g, device=dev)] += 20
    probs = torch.empty_like(lg)
    idx = torch.empty(64, dtype=torch.int32, device=dev)
    fl = torch.empty(64, dtype=torch.int32, device=dev)
    ws = K.rows_workspace(64, 128256, dev)
    timer = Timer(torch)
    out = {}
    items = {
        "add_rmsnorm_8192x4096": (lambda: K.add_rmsnorm(h, d, w, 1e-5, n), 4 * 8192 * 4096 * 2),
        "silu_mul_8192x14336": (lambda: K.silu_mul(act, gate, up), 3 * 8192 * 14336 * 2),
        "softmax_64x128256": (lambda: K.softmax_rows(lg, probs, 1.0, ws), 2 * 64 * 128256 * 4),
        "argmax_64x128256": (lambda: K.argmax_rows(lg, idx, fl, ws), 64 * 128256 * 4),
        "softmax_argmax_64x128256": (lambda: K.softmax_argmax_rows(lg, probs, idx, fl, 1.0, ws),
                                     2 * 64 * 128256 * 4),
    }
    for name, (fn, nb) in items.items():
        # the 64-row reductions run for less than the host needs to issue a call: time them
        # from a HIP graph so that the figure is the GPU's, not the launch path's
        if name.startswith(("softmax", "argmax")):
            us = timer.graph_time_us(fn)
        else:
            us = timer.time_us(fn, 50, warmup=5)
        out[name] = {"us": round(us, 2), "GB/s": round(gbs(nb, us), 1),
                     "frac_of_peak": round(gbs(nb, us) / PEAK_HBM_GBS, 4), "bytes": nb,
                     "traffic": traffic_of(name)}
    floors = run_floors(torch, K, dev)
    for name in ("softmax_64x128256", "argmax_64x128256"):
        with_floor(out[name], floors[name])
        out[name]["floor_cold_us"] = floors[name + "_cold"]["us"]
    return {"workload": "prefill-shaped reductions (fp16 in, fp32 accumulate)", "kernels": out}


def run_tq(args, torch, K, dev):
    from fracture_amd import turboquant as tq

    g = torch.Generator(device=dev)
    g.manual_seed(2)
    N, H, hd = 32768, 8, 128
    scale = torch.exp(torch.randn((N, 1, 1), generator=g, device=dev) * 0.5)
    k = (torch.randn((N, H, hd), generator=g, device=dev) * scale).to(torch.float16)
    v = (torch.randn((N, H, hd), generator=g, device=dev) * scale).to(torch.float16)
    krot = torch.from_numpy(tq.rotation_matrix(hd, 42)).to(dev)
    vrot = torch.from_numpy(tq.rotation_matrix(hd, 542)).to(dev)
    timer = Timer(torch)
    out = {}
    for bits in (4, 3):
        cent = torch.from_numpy(tq.codebook(hd, bits)[0]).to(dev)
        pd = K.packed_dim(hd, bits)
        kp = torch.empty((N, H * pd), dtype=torch.uint8, device=dev)
        vp = torch.empty_like(kp)
        kn = torch.empty((N, H), dtype=torch.float16, device=dev)
        vn = torch.empty_like(kn)
        kd = torch.empty_like(k)
        vd = torch.empty_like(v)

        # the per-layer plans (built once, as the cache manager uploads the rotations and
        # codebooks once) and the reference-signature entries that rebuild them per call
        kplan, vplan = K.TqPlan(krot, cent, bits), K.TqPlan(vrot, cent, bits)

        # the layer's keys and values in one launch (as append_kv compresses them)
        def comp():
            K.tq_compress_kv_planned(kplan, vplan, k, v, kp, kn, vp, vn)

        def deq():
            K.tq_dequant_kv_planned(kplan, vplan, kp, kn, vp, vn, kd, vd)

        # one launch per tensor (the trait's turboquant_compress per tensor, with a plan)
        def comp_split():
            K.tq_compress_planned(kplan, k, kp, kn)
            K.tq_compress_planned(vplan, v, vp, vn)

        def deq_split():
            K.tq_dequant_planned(kplan, kp, kn, kd)
            K.tq_dequant_planned(vplan, vp, vn, vd)

        def comp_unplanned():
            K.tq_compress(k, krot, cent, bits, kp, kn)
            K.tq_compress(v, vrot, cent, bits, vp, vn)

        def deq_unplanned():
            K.tq_dequant(kp, kn, krot, cent, bits, kd)
            K.tq_dequant(vp, vn, vrot, cent, bits, vd)

        nb = 2 * (N * H * hd * 2 + N * H * pd + N * H * 2)  # K and V: read fp16, write codes+norms
        flops = 2 * 2 * N * H * hd * hd
        for name, fn, tkey in (("compress", comp, "compress"), ("dequant", deq, "dequant"),
                               ("compress_per_tensor", comp_split, None),
                               ("dequant_per_tensor", deq_split, None),
                               ("compress_unplanned", comp_unplanned, None),
                               ("dequant_unplanned", deq_unplanned, None)):
            us = timer.time_us(fn, 20, warmup=3)
            out[f"tq_{name}_kv_{bits}bit"] = {
                "us": round(us, 2), "GB/s": round(gbs(nb, us), 1),
                "frac_of_peak": round(gbs(nb, us) / PEAK_HBM_GBS, 4), "bytes": nb,
                "rotation_TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1),
                "traffic": traffic_of(f"tq_{tkey}_{bits}bit") if tkey else None}
    return {"workload": "TurboQuant KV compress / dequantize, one layer, [32768, 8, 128] K and V",
            "kernels": out}


def prefill_attention_inputs(torch, K, dev, T, kv_len):
    """Causal prefill of T queries at positions kv_len - T .. kv_len - 1 of one sequence
    through the reference-signature launcher (per-page address arrays into one pool, K4/V4,
    32/8 heads): returns (fn, algorithmic bytes, positions scored per kv head)."""
    import ctypes as C

    import numpy as np

    from fracture_amd import turboquant as tq

    QH, KVH, HD = ATT_SHAPE["QH"], ATT_SHAPE["KVH"], ATT_SHAPE["HD"]
    nb = (kv_len + 15) // 16
    P = nb + 3
    g = torch.Generator(device=dev)
    g.manual_seed(T + kv_len)
    kp = torch.randint(0, 256, (P, 16, KVH * 64), generator=g, device=dev, dtype=torch.uint8)
    vp = torch.randint(0, 256, (P, 16, KVH * 64), generator=g, device=dev, dtype=torch.uint8)
    kn = (torch.rand((P, 16, KVH), generator=g, device=dev) * 10 + 6).to(torch.float16)
    vn = (torch.rand((P, 16, KVH), generator=g, device=dev) * 10 + 6).to(torch.float16)

    def ptrs(t, stride):
        return torch.tensor([t.data_ptr() + p * stride for p in range(P)], dtype=torch.int64,
                            device=dev)

    pk, pkn, pv, pvn = (ptrs(kp, 16 * KVH * 64), ptrs(kn, 16 * KVH * 2), ptrs(vp, 16 * KVH * 64),
                        ptrs(vn, 16 * KVH * 2))
    table = torch.from_numpy(np.random.default_rng(2).permutation(P)[:nb].astype(np.int32)).to(dev)
    q = torch.randn((T, QH, HD), generator=g, device=dev).to(torch.float16)
    out = torch.empty_like(q)
    krot = torch.from_numpy(tq.rotation_matrix(HD, 42)).to(dev)
    vrot = torch.from_numpy(tq.rotation_matrix(HD, 542)).to(dev)
    cent = torch.from_numpy(tq.codebook(HD, 4)[0]).to(dev)
    lib = K._L()
    wsb = lib.fhip_attention_tq_workspace_bytes(T, QH, HD, nb)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    keep = (kp, vp, kn, vn, pk, pkn, pv, pvn, table, q, out, krot, vrot, cent, ws)

    def fn():
        _ = keep
        r = lib.fhip_launch_attention_paged_tq_ws(
            out.data_ptr(), q.data_ptr(), table.data_ptr(), pk.data_ptr(), pkn.data_ptr(),
            pv.data_ptr(), pvn.data_ptr(), krot.data_ptr(), vrot.data_ptr(), cent.data_ptr(),
            cent.data_ptr(), T, QH, KVH, HD, kv_len, kv_len - T, 4, 4, 64, 64, ws.data_ptr(),
            C.c_size_t(wsb), K._stream())
        assert r == 0, r

    scored = sum(min(kv_len - T + t + 1, kv_len) for t in range(T))
    nbytes = kv_len * KVH * (64 + 64 + 4) + 2 * T * QH * HD * 2 + nb * 4
    return fn, nbytes, scored


def run_attention(args, torch, K, dev):
    fn, nb, tok, mean = attention_inputs(torch, K, dev)
    us = Timer(torch).time_us(fn, 10, warmup=2)
    kernels = {"attention_tq_decode": {
        "us": round(us, 1), "GB/s": round(gbs(nb, us), 1),
        "frac_of_peak": round(gbs(nb, us) / PEAK_HBM_GBS, 4), "bytes": nb,
        "context_tokens": tok, "mean_ctx": mean,
        "traffic": traffic_of("attention_tq_decode")}}
    fn, nb, _, _ = attention_inputs(torch, K, dev, vb=2)
    us = Timer(torch).time_us(fn, 10, warmup=2)
    kernels["attention_tq_decode_k4v2"] = {
        "us": round(us, 1), "GB/s": round(gbs(nb, us), 1),
        "frac_of_peak": round(gbs(nb, us) / PEAK_HBM_GBS, 4), "bytes": nb,
        "note": "the same batch with 2-bit V codes: K4/V2 is TurboQuantConfig's default"}
    del fn
    for T, kv_len in ((2048, 2048), (512, 8192)):
        pfn, pnb, scored = prefill_attention_inputs(torch, K, dev, T, kv_len)
        pus = Timer(torch).time_us(pfn, 5, warmup=2)
        kernels[f"attention_tq_prefill_T{T}_ctx{kv_len}"] = {
            "us": round(pus, 1), "GB/s": round(gbs(pnb, pus), 1),
            "frac_of_peak": round(gbs(pnb, pus) / PEAK_HBM_GBS, 5), "bytes": pnb,
            "positions_scored_per_kv_head": scored,
            "Gpos/s": round(scored * ATT_SHAPE["KVH"] / pus / 1e3, 2),
            "note": "causal prefill through fhip_launch_attention_paged_tq_ws; bytes are the "
                    "distinct K/V pages, queries and outputs (each page is re-read by every "
                    "group of 8 / G queries)"}
    return {"workload": "TurboQuant K4/V4 (and K4/V2) paged decode attention, B=64, 32/8 heads, "
                        "hd 128; causal prefill of one sequence", "kernels": kernels}


def paged_inputs(torch, K, dev):
    """FP16 paged decode attention at the same batch, heads and lengths as the TurboQuant
    workload: returns (fn, algorithmic bytes, context tokens, mean)."""
    import numpy as np

    B, QH, KVH, HD = (ATT_SHAPE[k] for k in ("B", "QH", "KVH", "HD"))
    lens = attention_lens()
    rng = np.random.default_rng(5)
    rng.integers(1024, 32769, B)
    nbs = (lens + 15) // 16
    P = int(nbs.sum())
    maxb = int(nbs.max())
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, maxb), np.int32)
    at = 0
    for b in range(B):
        table[b, :nbs[b]] = perm[at:at + nbs[b]]
        at += nbs[b]
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    kp = torch.randn((P, 16, KVH, HD), generator=g, device=dev, dtype=torch.float16)
    vp = torch.randn((P, 16, KVH, HD), generator=g, device=dev, dtype=torch.float16)
    q = torch.randn((B, QH, HD), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    tb = torch.from_numpy(table).to(dev)
    sl = torch.from_numpy(lens).to(dev)
    ws = K.attention_paged_workspace(B, QH, HD, maxb, dev)
    fn = lambda: K.attention_paged_decode(out, q, tb, sl, kp, vp, KVH, ws)
    tok = int(lens.sum())
    nb = tok * KVH * HD * 2 * 2 + 2 * B * QH * HD * 2 + B * maxb * 4
    return fn, nb, tok, float(lens.mean())


def paged_prefill_inputs(torch, K, dev, T, kv_len):
    """FP16 causal prefill of T queries at positions kv_len - T .. kv_len - 1 of one sequence
    through the reference-signature launcher (per-page address arrays, 32/8 heads, hd 128):
    returns (fn, algorithmic bytes, positions scored per kv head)."""
    import numpy as np

    QH, KVH, HD = ATT_SHAPE["QH"], ATT_SHAPE["KVH"], ATT_SHAPE["HD"]
    nb = (kv_len + 15) // 16
    P = nb + 3
    g = torch.Generator(device=dev)
    g.manual_seed(T + kv_len)
    kp = torch.randn((P, 16, KVH, HD), generator=g, device=dev, dtype=torch.float16)
    vp = torch.randn((P, 16, KVH, HD), generator=g, device=dev, dtype=torch.float16)
    kptr = torch.tensor([kp[i].data_ptr() for i in range(P)], dtype=torch.int64, device=dev)
    vptr = torch.tensor([vp[i].data_ptr() for i in range(P)], dtype=torch.int64, device=dev)
    table = torch.from_numpy(np.random.default_rng(2).permutation(P)[:nb].astype(np.int32)).to(dev)
    q = torch.randn((T, QH, HD), generator=g, device=dev).to(torch.float16)
    out = torch.empty_like(q)
    ws = K.attention_paged_workspace(T, QH, HD, nb, dev)
    fn = lambda: K.paged_attention(out, q, table, kptr, vptr, KVH, kv_len, kv_len - T, ws)
    scored = sum(min(kv_len - T + t + 1, kv_len) for t in range(T))
    nbytes = kv_len * KVH * HD * 2 * 2 + 2 * T * QH * HD * 2 + nb * 4
    return fn, nbytes, scored


def run_paged(args, torch, K, dev):
    fn, nb, tok, mean = paged_inputs(torch, K, dev)
    us = Timer(torch).time_us(fn, 10, warmup=2)
    kernels = {"attention_paged_decode": {
        "us": round(us, 1), "GB/s": round(gbs(nb, us), 1),
        "frac_of_peak": round(gbs(nb, us) / PEAK_HBM_GBS, 4), "bytes": nb,
        "context_tokens": tok, "mean_ctx": mean,
        "traffic": traffic_of("attention_paged_decode")}}
    for T, kv_len in ((2048, 2048), (512, 8192)):
        pfn, pnb, scored = paged_prefill_inputs(torch, K, dev, T, kv_len)
        pus = Timer(torch).time_us(pfn, 5, warmup=2)
        kernels[f"attention_paged_prefill_T{T}_ctx{kv_len}"] = {
            "us": round(pus, 1), "GB/s": round(gbs(pnb, pus), 1),
            "frac_of_peak": round(gbs(pnb, pus) / PEAK_HBM_GBS, 5), "bytes": pnb,
            "positions_scored_per_kv_head": scored,
            "Gpos/s": round(scored * ATT_SHAPE["KVH"] / pus / 1e3, 2),
            "note": "causal prefill through fhip_launch_paged_attention_ws; bytes are the "
                    "distinct K/V pages, queries and outputs (each page is re-read by every "
                    "group of 8 / G queries)"}
    return {"workload": "FP16 paged decode attention, B=64, 32/8 heads, hd 128; causal "
                        "prefill of one sequence", "kernels": kernels}


# ---------------------------------------------------------------------------------------
# HBM traffic from rocprofv3 PMC counters
# ---------------------------------------------------------------------------------------
CAL_BYTES = 1 << 30
ATT_SHAPE = dict(B=64, QH=32, KVH=8, HD=128, kb=4, vb=4)


def attention_inputs(torch, K, dev, vb=None):
    """The decode-attention workload (V codes of ATT_SHAPE's width unless vb is given): returns
    (fn, algorithmic bytes, context tokens, mean)."""
    import numpy as np

    from fracture_amd import turboquant as tq

    B, QH, KVH, HD, kb = (ATT_SHAPE[k] for k in ("B", "QH", "KVH", "HD", "kb"))
    vb = ATT_SHAPE["vb"] if vb is None else vb
    lens = attention_lens()
    rng = np.random.default_rng(5)
    rng.integers(1024, 32769, B)  # the lengths' draw: the page permutation comes next
    nbs = (lens + 15) // 16
    P = int(nbs.sum())
    maxb = int(nbs.max())
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, maxb), np.int32)
    at = 0
    for b in range(B):
        table[b, :nbs[b]] = perm[at:at + nbs[b]]
        at += nbs[b]
    pdk, pdv = K.packed_dim(HD, kb), K.packed_dim(HD, vb)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    kp = torch.randint(0, 256, (P, 16, KVH * pdk), generator=g, device=dev, dtype=torch.uint8)
    vp = torch.randint(0, 256, (P, 16, KVH * pdv), generator=g, device=dev, dtype=torch.uint8)
    kn = (torch.rand((P, 16, KVH), generator=g, device=dev) * 10 + 6).to(torch.float16)
    vn = (torch.rand((P, 16, KVH), generator=g, device=dev) * 10 + 6).to(torch.float16)
    q = torch.randn((B, QH, HD), generator=g, device=dev).to(torch.float16)
    out = torch.empty_like(q)
    krot = torch.from_numpy(tq.rotation_matrix(HD, 42)).to(dev)
    vrot = torch.from_numpy(tq.rotation_matrix(HD, 542)).to(dev)
    kc = torch.from_numpy(tq.codebook(HD, kb)[0]).to(dev)
    vc = torch.from_numpy(tq.codebook(HD, vb)[0]).to(dev)
    tb = torch.from_numpy(table).to(dev)
    sl = torch.from_numpy(lens).to(dev)
    ws = K.attention_workspace(B, QH, HD, maxb, dev)
    fn = lambda: K.attention_tq_decode(out, q, tb, sl, kp, kn, vp, vn, krot, vrot, kc, vc, kb, vb,
                                       KVH, ws)
    tok = int(lens.sum())
    nb = tok * KVH * (pdk + pdv + 4) + B * QH * HD * 4 + B * maxb * 4
    return fn, nb, tok, float(lens.mean())


def pmc_sequence(torch, K, dev):
    """[(key, fn, algorithmic bytes)] of every measured operation, inputs already resident."""
    from fracture_amd import turboquant as tq

    seq = []
    x = decode_inputs(torch, dev)
    ops = decode_ops(K, x)
    nb = decode_bytes()
    seq += [("decode_embedding", ops["embedding"], nb["embedding"]),
            ("decode_rope", ops["rope"], nb["rope"]),
            ("silu_mul_64x14336", ops["silu_mul"], nb["silu_mul"]),
            ("decode_add_rmsnorm", ops["add_rmsnorm"], nb["add_rmsnorm"])]
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    f16 = torch.float16
    h = torch.randn((8192, 4096), generator=g, device=dev).to(f16)
    d = torch.randn((8192, 4096), generator=g, device=dev).to(f16)
    w = (torch.rand((4096,), generator=g, device=dev) + 0.5).to(f16)
    n = torch.empty_like(h)
    gate = torch.randn((8192, 14336), generator=g, device=dev).to(f16)
    up = torch.randn((8192, 14336), generator=g, device=dev).to(f16)
    act = torch.empty_like(gate)
    lg = torch.randn((64, 128256), generator=g, device=dev) * 3
    probs = torch.empty_like(lg)
    idx = torch.empty(64, dtype=torch.int32, device=dev)
    fl = torch.empty(64, dtype=torch.int32, device=dev)
    ws = K.rows_workspace(64, 128256, dev)
    seq += [("add_rmsnorm_8192x4096", lambda: K.add_rmsnorm(h, d, w, 1e-5, n), 4 * 8192 * 4096 * 2),
            ("silu_mul_8192x14336", lambda: K.silu_mul(act, gate, up), 3 * 8192 * 14336 * 2),
            ("softmax_64x128256", lambda: K.softmax_rows(lg, probs, 1.0, ws), 2 * 64 * 128256 * 4),
            ("argmax_64x128256", lambda: K.argmax_rows(lg, idx, fl, ws), 64 * 128256 * 4),
            ("softmax_argmax_64x128256",
             lambda: K.softmax_argmax_rows(lg, probs, idx, fl, 1.0, ws), 2 * 64 * 128256 * 4)]
    N, H, hd = 32768, 8, 128
    kv = [(torch.randn((N, H, hd), generator=g, device=dev)).to(f16) for _ in range(2)]
    rots = [torch.from_numpy(tq.rotation_matrix(hd, s)).to(dev) for s in (42, 542)]
    for bits in (4, 3):
        cent = torch.from_numpy(tq.codebook(hd, bits)[0]).to(dev)
        pd = K.packed_dim(hd, bits)
        pk = [torch.empty((N, H * pd), dtype=torch.uint8, device=dev) for _ in range(2)]
        nm = [torch.empty((N, H), dtype=f16, device=dev) for _ in range(2)]
        dq = [torch.empty_like(kv[0]) for _ in range(2)]
        nbytes = 2 * (N * H * hd * 2 + N * H * pd + N * H * 2)

        plans = [K.TqPlan(rots[i], cent, bits) for i in range(2)]

        def comp(plans=plans, pk=pk, nm=nm):  # keys and values in one launch
            K.tq_compress_kv_planned(plans[0], plans[1], kv[0], kv[1], pk[0], nm[0], pk[1], nm[1])

        def deq(plans=plans, pk=pk, nm=nm, dq=dq):
            K.tq_dequant_kv_planned(plans[0], plans[1], pk[0], nm[0], pk[1], nm[1], dq[0], dq[1])

        seq += [(f"tq_compress_{bits}bit", comp, nbytes), (f"tq_dequant_{bits}bit", deq, nbytes)]
    fn, nb_att, _, _ = attention_inputs(torch, K, dev)
    seq.append(("attention_tq_decode", fn, nb_att))
    fn, nb_pg, _, _ = paged_inputs(torch, K, dev)
    seq.append(("attention_paged_decode", fn, nb_pg))
    return seq


def attention_lens():
    import numpy as np

    rng = np.random.default_rng(5)
    return rng.integers(1024, 32769, ATT_SHAPE["B"]).astype(np.int32)


def pmc_keys():
    """[(key, algorithmic bytes)] of pmc_sequence(), computed without a GPU."""
    nb = decode_bytes()
    keys = [("decode_embedding", nb["embedding"]), ("decode_rope", nb["rope"]),
            ("silu_mul_64x14336", nb["silu_mul"]), ("decode_add_rmsnorm", nb["add_rmsnorm"]),
            ("add_rmsnorm_8192x4096", 4 * 8192 * 4096 * 2),
            ("silu_mul_8192x14336", 3 * 8192 * 14336 * 2),
            ("softmax_64x128256", 2 * 64 * 128256 * 4), ("argmax_64x128256", 64 * 128256 * 4),
            ("softmax_argmax_64x128256", 2 * 64 * 128256 * 4)]
    N, H, hd = 32768, 8, 128
    for bits in (4, 3):
        pd = (hd * bits + 7) // 8
        nbytes = 2 * (N * H * hd * 2 + N * H * pd + N * H * 2)
        keys += [(f"tq_compress_{bits}bit", nbytes), (f"tq_dequant_{bits}bit", nbytes)]
    lens = attention_lens()
    a = ATT_SHAPE
    maxb = int(((lens + 15) // 16).max())
    pdk, pdv = a["HD"] * a["kb"] // 8, a["HD"] * a["vb"] // 8
    keys.append(("attention_tq_decode", int(lens.sum()) * a["KVH"] * (pdk + pdv + 4) +
                 a["B"] * a["QH"] * a["HD"] * 4 + a["B"] * maxb * 4))
    keys.append(("attention_paged_decode", int(lens.sum()) * a["KVH"] * a["HD"] * 4 +
                 2 * a["B"] * a["QH"] * a["HD"] * 2 + a["B"] * maxb * 4))
    return keys


def runtime_attention_inputs(torch, K, dev):
    """The decode-attention workload as the engine drives it through the handle runtime: one
    (K packed, K norms, V packed, V norms) tensor per block, registered as a pool, filled with
    append_kv per sequence; the call is fhip_attention_paged_tq_batched. Returns (fn, bytes,
    cleanup)."""
    import numpy as np

    from fracture_amd import DType, HipBackend
    from fracture_amd import turboquant as tq

    B, QH, KVH, HD = (ATT_SHAPE[k] for k in ("B", "QH", "KVH", "HD"))
    lens = attention_lens()
    rng = np.random.default_rng(5)
    rng.integers(1024, 32769, B)
    nbs = (lens + 15) // 16
    P = int(nbs.sum())
    perm = rng.permutation(P)
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at:at + nb].tolist())
        at += nb
    be = HipBackend(0)
    lists = [[be.alloc(shape, dt) for _ in range(P)] for shape, dt in
             (([16, KVH * 64], DType.INT8), ([16, KVH], DType.FP16),
              ([16, KVH * 64], DType.INT8), ([16, KVH], DType.FP16))]
    pool = be.page_pool_create(*lists)
    krot, vrot = tq.rotation_matrix(HD, 42), tq.rotation_matrix(HD, 542)
    cent = tq.codebook(HD, 4)[0]
    tkr, tvr, tc = (be.upload(a) for a in (krot, vrot, cent))
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    zeros = torch.zeros((int(lens.max()), KVH, HD), dtype=torch.float16, device=dev)
    for b in range(B):
        n = int(lens[b])
        ts = []
        for _ in range(2):
            x = torch.randn((n, KVH, HD), generator=g, device=dev).to(torch.float16)
            t = be.alloc([n, KVH, HD], DType.FP16)
            # the backend tensor = x + 0 (a device copy, on torch's stream)
            assert K._L().fhip_launch_add_ex(be.get_ptr(t.id), x.data_ptr(), zeros.data_ptr(),
                                             x.numel(), 0, K._stream()) == 0
            torch.cuda.synchronize()
            ts.append(t)
        be.tq_append_kv(pool, ts[0], ts[1], tkr, tvr, tc, tc, 4, 4, tables[b], 0)
        for t in ts:
            be.free(t)
    q = be.upload(rng.standard_normal((B, QH, HD)).astype(np.float16))
    out = be.alloc([B, QH, HD], DType.FP16)
    table = np.full((B, int(nbs.max())), -1, np.int32)
    for b, row in enumerate(tables):
        table[b, :len(row)] = row
    lens_u = lens.astype(np.uint32)
    fn = lambda: be.attention_paged_tq_batched(q, table, lens_u, pool, tkr, tvr, tc, tc, 4, 4,
                                               KVH, out)
    tok = int(lens.sum())
    nb = tok * KVH * (64 + 64 + 4) + B * QH * HD * 4 + B * int(nbs.max()) * 4

    def cleanup():
        be.synchronize()
        be.page_pool_destroy(pool)
        be.close()  # frees every tensor at once

    return fn, nb, cleanup, be


def kernel_entry(us, nb, **extra):
    e = {"us": round(us, 2), "GB/s": round(gbs(nb, us), 1),
         "frac_of_peak": round(gbs(nb, us) / PEAK_HBM_GBS, 4), "bytes": nb}
    e.update(extra)
    return e


def run_configs(args, torch, K, dev):
    """Compact results of the other configurations for the default JSON line."""
    out = {}
    pre = run_prefill(args, torch, K, dev)["kernels"]
    out["c3_prefill_reductions"] = {k: {f: v[f] for f in ("us", "GB/s", "frac_of_peak",
                                                          "floor_us", "frac_of_floor") if f in v}
                                    for k, v in pre.items()}
    tqr = run_tq(args, torch, K, dev)["kernels"]
    out["c4_turboquant_kv_32768x8x128"] = {
        k: {f: v[f] for f in ("us", "GB/s", "frac_of_peak", "rotation_TFLOP/s")}
        for k, v in tqr.items()}
    att = run_attention(args, torch, K, dev)["kernels"]["attention_tq_decode"]
    c5 = {"contiguous_pools": {f: att[f] for f in ("us", "GB/s", "frac_of_peak")}}
    fn, nb, cleanup, be = runtime_attention_inputs(torch, K, dev)
    # each call stages its block table and lengths through 2 of the backend's 16 pinned slots,
    # which are allocated on first use: warm up past one turn of the ring
    # (and past the clock ramp: ~100 calls of ~0.4 ms)
    for _ in range(100):
        fn()
    be.synchronize()
    reps = 20
    tm = be.create_timer()
    gpu, host = [], []
    for _ in range(5):
        t0 = time.perf_counter()
        be.start_timer(tm)
        for _ in range(reps):
            fn()
        gpu.append(be.stop_timer(tm) * 1e3 / reps)  # HIP events on the backend's stream
        be.synchronize()
        host.append((time.perf_counter() - t0) * 1e6 / reps)
    be.destroy_timer(tm)
    gpu_us, us = sorted(gpu)[2], sorted(host)[2]
    c5["handle_runtime_per_block_tensors"] = dict(
        kernel_entry(gpu_us, nb), host_us_per_call=round(us, 1),
        note="fhip_attention_paged_tq_batched over a registered pool of per-block tensors "
             "filled by fhip_tq_append_kv: HIP events on the backend stream; host_us_per_call "
             "is the wall time per call (block-table staging and checks included)")
    cleanup()
    out["c5_tq_decode_attention_B64_K4V4"] = c5
    return out


def cpu_config_baselines(seconds: float):
    """The oracle on this host for the other configurations: one thread and all cores, each on
    a bounded sample of the workload, scaled to the full workload's size."""
    import numpy as np

    import oracle
    from fracture_amd import turboquant as tq

    th = cpu_threads()
    rng = np.random.default_rng(0)
    out = {}

    def both(fn1, fnN, scale, nbytes, sample):
        t1, _ = median_time(fn1, 3, seconds)
        tN, _ = median_time(fnN, 3, seconds)
        return {"us_1core": round(t1 * scale * 1e6, 1), "us_all_cores": round(tN * scale * 1e6, 1),
                "GB/s_1core": round(gbs(nbytes, t1 * scale * 1e6), 3),
                "GB/s_all_cores": round(gbs(nbytes, tN * scale * 1e6), 3), "sample": sample}

    # the CPU configuration itself: fp32 add + RMSNorm on [32, 4096], X and the residual
    # ~N(0,1), weight ~U(0.5,1.5), seed 0, eps 1e-5 (the whole workload, no scaling)
    r1 = np.random.default_rng(0)
    x1 = r1.standard_normal((32, 4096)).astype(np.float32)
    res1 = r1.standard_normal((32, 4096)).astype(np.float32)
    w1 = r1.uniform(0.5, 1.5, 4096).astype(np.float32)
    out["c1_add_rmsnorm_fp32_32x4096"] = both(
        lambda: oracle.add_rmsnorm(res1, x1, w1, 1e-5),
        lambda: par_rows(lambda a, b: oracle.add_rmsnorm(a, b, w1, 1e-5), [res1, x1], 32, th),
        1.0, 4 * 32 * 4096 * 4 + 4096 * 4, "the whole workload (32 rows)")

    R = 512
    h = rng.standard_normal((R, 4096)).astype(np.float16)
    d = rng.standard_normal((R, 4096)).astype(np.float16)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float16)
    gt = rng.standard_normal((R, 14336)).astype(np.float16)
    up = rng.standard_normal((R, 14336)).astype(np.float16)
    lg = (rng.standard_normal((64, 128256)) * 3).astype(np.float32)
    lg[np.arange(64), rng.integers(0, 128256, 64)] += 20
    c3 = {}
    c3["add_rmsnorm_8192x4096"] = both(
        lambda: oracle.add_rmsnorm(h, d, w, 1e-5),
        lambda: par_rows(lambda a, b: oracle.add_rmsnorm(a, b, w, 1e-5), [h, d], R, th),
        8192 / R, 4 * 8192 * 4096 * 2, f"{R} of 8192 rows")
    c3["silu_mul_8192x14336"] = both(
        lambda: oracle.silu_mul(gt, up), lambda: par_rows(oracle.silu_mul, [gt, up], R, th),
        8192 / R, 3 * 8192 * 14336 * 2, f"{R} of 8192 rows")
    c3["softmax_64x128256"] = both(
        lambda: oracle.softmax_rows(lg), lambda: par_rows(oracle.softmax_rows, [lg], 64, th),
        1.0, 2 * 64 * 128256 * 4, "all 64 rows")
    c3["argmax_64x128256"] = both(
        lambda: oracle.argmax_rows(lg), lambda: par_rows(oracle.argmax_rows, [lg], 64, th),
        1.0, 64 * 128256 * 4, "all 64 rows")
    out["c3_prefill_reductions"] = c3

    N, H, hd = 512, 8, 128
    x = (rng.standard_normal((N, H, hd)) * np.exp(rng.normal(0, 0.5, (N, 1, 1)))).astype(np.float16)
    rot = tq.rotation_matrix(hd, 42)
    c4 = {}
    for bits in (4, 3):
        cent = tq.codebook(hd, bits)[0]
        pd = (hd * bits + 7) // 8
        pk, nm, _ = oracle.tq_compress(x, rot, cent, bits)
        nb = 2 * (32768 * H * hd * 2 + 32768 * H * pd + 32768 * H * 2)
        scale = 2 * 32768 / N  # K and V of 32768 tokens
        c4[f"tq_compress_kv_{bits}bit"] = both(
            lambda: oracle.tq_compress(x, rot, cent, bits),
            lambda: par_rows(lambda a: oracle.tq_compress(a, rot, cent, bits), [x], N, th),
            scale, nb, f"{N} tokens x 8 heads, scaled to K and V of 32768 tokens")
        nmf = nm.reshape(N, H)
        pkr = pk.reshape(N, H * pd)
        c4[f"tq_dequant_kv_{bits}bit"] = both(
            lambda: oracle.tq_dequant(pkr, nmf, rot, cent, bits, hd),
            lambda: par_rows(lambda a, b: oracle.tq_dequant(a, b, rot, cent, bits, hd),
                             [pkr, nmf], N, th),
            scale, nb, f"{N} tokens x 8 heads, scaled to K and V of 32768 tokens")
    out["c4_turboquant_kv_32768x8x128"] = c4

    # decode attention: 2 sequences x one query head per kv head, per (position, head) time
    # scaled to the workload's total context x 32 heads
    lens_s = [16384, 8192]
    nbs = [n // 16 for n in lens_s]
    P = sum(nbs)
    kp = rng.integers(0, 256, (P, 16, 8 * 64)).astype(np.uint8)
    vp = rng.integers(0, 256, (P, 16, 8 * 64)).astype(np.uint8)
    kn = rng.uniform(6, 16, (P, 16, 8)).astype(np.float16)
    vn = rng.uniform(6, 16, (P, 16, 8)).astype(np.float16)
    perm = rng.permutation(P).astype(np.int32)
    tabs = [perm[:nbs[0]], perm[nbs[0]:]]
    q = rng.standard_normal((32, 128)).astype(np.float16)
    krot, vrot = tq.rotation_matrix(128, 42), tq.rotation_matrix(128, 542)
    cent = tq.codebook(128, 4)[0]
    jobs = [(i, 4 * g_) for i in range(2) for g_ in range(8)]

    def one(job):
        i, h0 = job
        oracle.tq_attention(q, tabs[i], lens_s[i], kp, kn, vp, vn, krot, vrot, cent, cent, 4, 4,
                            8, heads=(h0, h0 + 1))

    def serial():
        for j in jobs:
            one(j)

    def parallel():
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(th) as ex:
            list(ex.map(one, jobs))

    lens = attention_lens()
    work = float(lens.sum()) * 32
    done = float(sum(lens_s)) * 8
    nb = int(lens.sum()) * 8 * (64 + 64 + 4) + 64 * 32 * 128 * 4 + 64 * int(((lens + 15) // 16).max()) * 4
    out["c5_tq_decode_attention_B64_K4V4"] = both(
        serial, parallel, work / done, nb,
        "2 sequences (16384 and 8192 positions) x 8 query heads, scaled to the workload's "
        "total context x 32 heads")
    return out


def run_pmc(torch, K, dev):
    seq = pmc_sequence(torch, K, dev)
    assert [(k, nb) for k, _, nb in seq] == pmc_keys(), "pmc_keys() out of step"
    for _, fn, _ in seq:  # first calls (lazy set-up) outside the counted sequence
        fn()
    big_a = torch.ones(CAL_BYTES, dtype=torch.uint8, device=dev)
    big_b = torch.empty_like(big_a)
    mark_a = torch.ones(4096, dtype=torch.uint8, device=dev)
    mark_b = torch.empty_like(mark_a)
    torch.cuda.synchronize()
    big_b.copy_(big_a)
    for _, fn, _ in seq:
        mark_b.copy_(mark_a)
        fn()
    mark_b.copy_(mark_a)
    torch.cuda.synchronize()
    return {"pmc_sequence": [(k, nb) for k, _, nb in seq], "calibration_bytes": CAL_BYTES}


def _pmc_rows(directory: str, counter: str):
    """(dispatch id, kernel name, value) of one counter, in dispatch order."""
    import glob
    import sqlite3

    dbs = sorted(glob.glob(os.path.join(directory, "**", "*_results.db"), recursive=True))
    if not dbs:
        raise SystemExit(f"no rocpd database under {directory}")
    rows = []
    for db in dbs:
        c = sqlite3.connect(db)
        rows += c.execute("select dispatch_id, kernel_name, value from counters_collection "
                          "where counter_name = ?", (counter,)).fetchall()
    rows.sort()
    return rows


def traffic_from(fetch_dir: str, write_dir: str, keys):
    """Per-operation HBM bytes: counter readings between marker copies, scaled by the
    counters' reading for the 1 GiB calibration copy."""
    out = {}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _pmc_rows(directory, counter)
        copies = [i for i, r in enumerate(rows) if "copyBuffer" in r[1]]
        if len(copies) < len(keys) + 2:
            raise SystemExit(f"{counter}: expected {len(keys) + 2} marker copies, "
                             f"found {len(copies)}")
        cal, marks = copies[-(len(keys) + 2)], copies[-(len(keys) + 1):]
        factor = rows[cal][2] * 1024.0 / CAL_BYTES  # counter KiB per true KiB
        for j, (key, nb) in enumerate(keys):
            seg = rows[marks[j] + 1:marks[j + 1]]
            e = out.setdefault(key, {"algorithmic_bytes": nb})
            e[counter.lower() + "_bytes"] = round(sum(r[2] for r in seg) * 1024.0 / factor)
            e[counter.lower() + "_counter_per_byte"] = round(factor, 4)
            e["dispatches"] = len(seg)
    for e in out.values():
        e["bytes_per_dispatch"] = e["fetch_size_bytes"] + e["write_size_bytes"]
        e["traffic_over_algorithmic"] = round(e["bytes_per_dispatch"] / e["algorithmic_bytes"], 3)
    return out


def ktrace_summary(directory: str, min_run: int = 50) -> str:
    """Markdown table of a `rocprofv3 --kernel-trace` run: this library's kernels grouped by
    name and grid, with the dispatches that ran in back-to-back runs of at least `min_run`
    (the HIP graphs the per-kernel timings replay) summarised on their own."""
    import re
    import sqlite3
    import statistics

    dbs = sorted(Path(directory).rglob("*.db"))
    if not dbs:
        raise SystemExit(f"no rocpd database under {directory}")
    rows = []
    for db in dbs:
        c = sqlite3.connect(db)
        rows += c.execute("select name, start, end, grid_x, grid_y, workgroup_x, vgpr_count, "
                          "accum_vgpr_count, lds_size from kernels").fetchall()
    rows.sort(key=lambda r: r[1])
    # back-to-back runs: consecutive dispatches of one kernel and grid
    in_run = [False] * len(rows)
    i = 0
    while i < len(rows):
        j = i
        while j + 1 < len(rows) and rows[j + 1][0] == rows[i][0] and rows[j + 1][3:5] == rows[i][3:5]:
            j += 1
        if j - i + 1 >= min_run:
            for k in range(i, j + 1):
                in_run[k] = True
        i = j + 1
    groups, meta = {}, {}
    for r, b2b in zip(rows, in_run):
        name = r[0]
        if "at::" in name or "rocclr" in name or "elementwise_kernel" in name:
            continue
        short = re.sub(r"\(.*", "", name.replace("void ", "").replace("(anonymous namespace)::", ""))
        key = (short, r[3], r[4])
        groups.setdefault(key, []).append(((r[2] - r[1]) / 1e3, b2b))
        meta[key] = r[5:]
    # a kernel launched over many grid sizes (per-sequence copies) collapses into one row
    by_name = {}
    for key in groups:
        by_name.setdefault(key[0], []).append(key)
    for name, keys in by_name.items():
        if len(keys) > 4:
            merged = [d for k in keys for d in groups.pop(k)]
            groups[(name, f"{len(keys)} grids", "")] = merged
            meta[(name, f"{len(keys)} grids", "")] = meta[keys[0]]
    lines = [f"| kernel | calls | avg µs | median µs | min µs | max µs | grid x | grid y | block "
             f"| VGPR | AGPR | LDS B | calls in runs of >= {min_run} | their avg µs |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for key, d in sorted(groups.items(), key=lambda kv: -sum(x for x, _ in kv[1])):
        us = [x for x, _ in d]
        run = [x for x, b in d if b]
        wx, vg, ag, lds = meta[key]
        lines.append(f"| `{key[0]}` | {len(us)} | {sum(us) / len(us):.2f} | "
                     f"{statistics.median(us):.2f} | {min(us):.2f} | {max(us):.2f} | {key[1]} | "
                     f"{key[2]} | {wx} | {vg} | {ag} | {lds} | {len(run)} | "
                     + (f"{sum(run) / len(run):.2f} |" if run else "- |"))
    return "\n".join(lines)


def counters_summary(directories) -> str:
    """Markdown table of rocprofv3 --pmc runs (one directory per pass): each counter's value
    per dispatch (summed over the hardware instances the profiler reports), averaged over the
    dispatches of each of this library's kernels."""
    import re
    import sqlite3

    per = {}       # kernel -> counter -> [values per dispatch]
    order = []
    for d in directories:
        dbs = sorted(Path(d).rglob("*_results.db"))
        if not dbs:
            raise SystemExit(f"no rocpd database under {d}")
        for db in dbs:
            c = sqlite3.connect(db)
            rows = c.execute("select dispatch_id, kernel_name, counter_name, sum(value) from "
                             "counters_collection group by dispatch_id, counter_name").fetchall()
            for _, name, counter, value in rows:
                if "at::" in name or "rocclr" in name or "elementwise_kernel" in name:
                    continue
                short = re.sub(r"\(.*", "", name.replace("void ", "")
                               .replace("(anonymous namespace)::", ""))
                per.setdefault(short, {}).setdefault(counter, []).append(value)
                if counter not in order:
                    order.append(counter)
    lines = ["| kernel | dispatches | " + " | ".join(order) + " |",
             "|---|---|" + "---|" * len(order)]
    for k, cs in sorted(per.items()):
        n = max(len(v) for v in cs.values())
        cells = [f"{sum(cs[c]) / len(cs[c]):.4g}" if c in cs else "-" for c in order]
        lines.append(f"| `{k}` | {n} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def main():
    args = parse()
    if args.counters_from:
        print(counters_summary(args.counters_from))
        return
    if args.ktrace_from:
        print(ktrace_summary(args.ktrace_from))
        return
    if args.traffic_from:
        keys = pmc_keys()
        t = traffic_from(args.traffic_from[0], args.traffic_from[1], keys)
        (ROOT / "profiles" / "traffic.json").write_text(json.dumps(t, indent=1) + "\n")
        print("| operation | dispatches | fetch MB | write MB | HBM MB | algorithmic MB | ratio |")
        print("|---|---|---|---|---|---|---|")
        for k, e in t.items():
            print(f"| `{k}` | {e['dispatches']} | {e['fetch_size_bytes'] / 1e6:.2f} | "
                  f"{e['write_size_bytes'] / 1e6:.2f} | {e['bytes_per_dispatch'] / 1e6:.2f} | "
                  f"{e['algorithmic_bytes'] / 1e6:.2f} | {e['traffic_over_algorithmic']} |")
        return
    if args.gpus != 1:
        print(json.dumps({"error": "fracture_amd benchmarks one GPU: this build has no "
                                   "multi-GPU path; run with --gpus 1"}))
        sys.exit(2)
    import torch

    from fracture_amd import kernels as K

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    wl = args.workload
    if wl == "decode":
        res = run_decode(args, torch, K, dev)
        if not args.no_configs:
            res["configs"] = run_configs(args, torch, K, dev)
            if not args.no_cpu_baseline:
                res["cpu_baseline"]["configs"] = cpu_config_baselines(args.cpu_seconds / 40)
        print(json.dumps(res), flush=True)
    if wl == "all":
        print(json.dumps(run_decode(args, torch, K, dev)), flush=True)
    if wl in ("prefill", "all"):
        print(json.dumps(run_prefill(args, torch, K, dev)), flush=True)
    if wl in ("tq", "all"):
        print(json.dumps(run_tq(args, torch, K, dev)), flush=True)
    if wl in ("attention", "all"):
        print(json.dumps(run_attention(args, torch, K, dev)), flush=True)
    if wl in ("paged", "all"):
        print(json.dumps(run_paged(args, torch, K, dev)), flush=True)
    if wl in ("floors", "all"):
        print(json.dumps({"workload": "floors: empty kernel and traffic-only probes",
                          "floors": run_floors(torch, K, dev)}), flush=True)
    if wl == "pmc":
        print(json.dumps(run_pmc(torch, K, dev)), flush=True)


if __name__ == "__main__":
    main()
