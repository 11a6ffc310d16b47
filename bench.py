"""Benchmark of the TQ1_G128 hot path on one MI355X.

Headline workload: the decode GEMV at M=1 over the
three 27B-class matrices -- gate/up 5120->17408, down 17408->5120, QKV
5120->8192 -- with fp16 activations and fp32 accumulation. One *step* is one
GEMV over each of the three matrices. Weights are synthetic (BASELINE
distributions) and rotate through a ring of distinct copies larger than the
256 MiB Infinity Cache, so every launch streams its weights from HBM ("cold").
Inputs are resident in HBM before the timed region starts.

``value`` = packed weight bytes per step / wall time per step (events around
the whole timed region, launch gaps included). ``roofline`` is for the dominant
kernel (the gate/up GEMV): packed bytes per launch / its average launch
duration, from HIP events on the launch stream around `steps` cold launches
replayed back to back from one graph; ``traffic`` is the HBM bytes per launch
from the calibrated rocprofv3 --pmc passes recorded under profiles/. Secondary
figures: the 4096 x 4096 GEMV (configs[0], cold and warm), the small-batch GEMM
(configs[2], M=2..64, GB/s), the prefill GEMM
(configs[3], M=512 and 2048, TFLOP/s against the fp16 MFMA peak), the 64-layer
weight stream with one embedding row, and the reference's CPU
decode+matmul path (the oracle restatement) timed on the host cores on a
bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s

C0_K = C0_N = 4096  # configs[0]
C1_SHAPES = (("gate_up", 5120, 17408), ("down", 17408, 5120), ("qkv", 5120, 8192))  # (name, K, N)
C3_SHAPES = (("gate_up", 5120, 17408), ("down", 17408, 5120))
SMALL_BATCHES = (2, 4, 8, 16, 32, 64)
PREFILL_BATCHES = (512, 2048)
RING_BYTES_MIN = 600 * 1024 * 1024  # > 2 x (256 MiB MALL + L2)
RING_COPIES_MIN = 16                # and at least this many distinct copies


def ring_copies(matrix_bytes: int) -> int:
    """Distinct copies a cold ring of one matrix needs."""
    return max(RING_COPIES_MIN, -(-RING_BYTES_MIN // matrix_bytes))


def m1_form(handle, rows: int, columns: int) -> str:
    """The M=1 form the automatic configuration runs, read from its workspace
    query (from 2048 rows): none for the strip GEMV, the 64 KiB counter region
    alone for its K-chunk form, counters and partials for the (tile, group)
    LUT23 kernel."""
    ws = handle.ternel_tq1_matmul_workspace_bytes(1, rows, columns, 0, 0)
    if rows >= 2048 and ws == 0:
        return "strip"
    if rows >= 2048 and ws == 64 * 1024:
        return f"strip, {-(-columns // 128 // 40)} K chunks"
    return "lut23"


def packed_bytes(K: int, N: int) -> int:
    return N * (K // 128) * 28


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-model-stream", action="store_true")
    p.add_argument("--no-small-batch", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--stream-ceiling", action="store_true",
                   help="measure the single-launch HBM read ceiling (libternel_probe.so) at the configs' matrix "
                        "sizes and print one JSON line")
    p.add_argument("--phase-profile", action="store_true",
                   help="load the phase-timestamp build of the engine and summarise where a cold M=1 GEMV "
                        "launch spends its time, per configs[1] matrix (one JSON line each), next to the "
                        "graph-timed stream GEMV and LUT23 kernel")
    p.add_argument("--phase-batch", type=int, default=1,
                   help="activation rows of the --phase-profile launches: 1 profiles the LUT23 GEMV, more the "
                        "kernel the library's dispatch picks for that batch (stamped: the direct-fragment and wide forms)")
    p.add_argument("--prefill-probe", action="store_true",
                   help="run only the M=512 prefill GEMMs (gate/up, down), 2 warm-up + --steps eager launches "
                        "each, for rocprofv3 --pmc MFMA-utilisation passes")
    p.add_argument("--traffic-batch", type=int, default=1,
                   help="activation rows of the --traffic-probe launches (the library's dispatch for that batch)")
    p.add_argument("--traffic-probe", action="store_true",
                   help="only launch the dominant kernel eagerly over the cold ring, then a plain copy of "
                        "COPY_BYTES, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    p.add_argument("--dense-reference", action="store_true",
                   help="time the dense fp16 product of the same shapes through torch.mm (the vendor BLAS) at "
                        "M = 1, 16, 512 and 2048, for comparison with the packed kernels, one JSON line each")
    p.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                   help="summarise a rocprofv3 kernel_trace.csv per (kernel, grid) and exit")
    return p.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        counts = [i.get("num_threads", 0) for i in threadpool_info() if i.get("user_api") == "blas"]
        if counts:
            return int(max(counts))
    except Exception:
        pass
    return os.cpu_count() or 1


def timed_calls(fn, seconds: float, min_calls: int = 1) -> tuple[int, float]:
    """Calls fn() until `seconds` have elapsed (at least min_calls): (calls, elapsed s)."""
    calls = 0
    start = time.perf_counter()
    while True:
        fn()
        calls += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds and calls >= min_calls:
            return calls, elapsed


def cpu_baseline(seconds: float) -> dict:
    """The reference's CPU path, restated in the oracle, timed on a bounded sample
    whole gate/up decode + fp32 numpy matvec (the reported
    value, about half of `seconds`), the matvec alone over the pre-decoded matrix,
    and at configs[0] (4096 x 4096) decode + matvec and the literal per-row
    _reference_gemv restatement (src/bonsai_tq1/reference.py:14-65)."""
    import numpy as np

    from oracle import tq1_oracle as O
    from ternel_amd import synthetic

    name, K, N = C1_SHAPES[0]
    blocks = synthetic.host_blocks(N, K, seed=synthetic.SEED_BASE + 1)
    x = synthetic.host_activations(1, K, seed=synthetic.SEED_BASE + 1)
    calls, elapsed = timed_calls(lambda: O.cpu_decode_matmul(blocks, x, rows=N, columns=K), 0.5 * seconds)
    per_call = elapsed / calls
    dense = O.cpu_decode(blocks, rows=N, columns=K)
    mm_calls, mm_elapsed = timed_calls(lambda: O.cpu_matmul(dense, x), 0.15 * seconds)
    del dense, blocks

    K0, N0 = C0_K, C0_N
    blocks0 = synthetic.host_blocks(N0, K0, seed=synthetic.SEED_BASE + 0)
    x0 = synthetic.host_activations(1, K0, seed=synthetic.SEED_BASE + 0)
    c0_calls, c0_elapsed = timed_calls(lambda: O.cpu_decode_matmul(blocks0, x0, rows=N0, columns=K0), 0.15 * seconds)
    g0_calls, g0_elapsed = timed_calls(
        lambda: O.reference_gemv(blocks0, x0[0].astype(np.float32), rows=N0, columns=K0), 0.2 * seconds)
    bytes0 = packed_bytes(K0, N0)
    return {
        "value": round(packed_bytes(K, N) / per_call / 1e9, 4),
        "unit": "GB/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": (f"{calls} x full decode (oracle decode_tq1_blocks restatement) + fp32 numpy matvec of the "
                   f"{name} matrix K={K} N={N} ({packed_bytes(K, N)} packed bytes), {elapsed:.1f} s; "
                   f"decode is single-threaded numpy, the matvec uses the BLAS threads"),
        "seconds_per_call": round(per_call, 4),
        "matmul_only": {"calls": mm_calls, "ms_per_call": round(mm_elapsed / mm_calls * 1e3, 3),
                        "packed_GB/s": round(packed_bytes(K, N) / (mm_elapsed / mm_calls) / 1e9, 3),
                        "dense_fp32_GB/s": round(4 * K * N / (mm_elapsed / mm_calls) / 1e9, 2),
                        "what": f"fp32 numpy matvec over the pre-decoded dense {name} W (BLAS threads)"},
        "config0": {"workload": "configs[0]: M=1, K=N=4096, fp16 activations",
                    "decode_matmul_ms": round(c0_elapsed / c0_calls * 1e3, 2),
                    "decode_matmul_GB/s": round(bytes0 / (c0_elapsed / c0_calls) / 1e9, 4),
                    "reference_gemv_ms": round(g0_elapsed / g0_calls * 1e3, 2),
                    "reference_gemv_GB/s": round(bytes0 / (g0_elapsed / g0_calls) / 1e9, 4),
                    "calls": {"decode_matmul": c0_calls, "reference_gemv": g0_calls},
                    "reference_gemv_is": "per-row decode, fp32 group dots, fp32 scale sum, single-threaded"},
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def is_engine_kernel(name: str) -> bool:
    """The library's kernels (anonymous-namespace symbols) and the runtime's copy blit."""
    return "_GLOBAL__N_" in name or name.startswith("(anonymous namespace)::") or name == "__amd_rocclr_copyBuffer"


def trace_summary(path: str) -> int:
    """Per-(kernel, grid) launch statistics of the engine's kernels from a rocprofv3
    kernel_trace.csv (the kernel statistics file groups every grid of one template
    instance together); torch's kernels of the synthetic-data setup are left out."""
    import csv
    import statistics

    groups: dict = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if not is_engine_kernel(row["Kernel_Name"]):
                continue
            key = (row["Kernel_Name"], row["Grid_Size_X"], row["Grid_Size_Y"], row["Grid_Size_Z"])
            groups.setdefault(key, []).append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    print(f"{'calls':>6} {'avg_us':>9} {'p5_us':>8} {'median_us':>9} {'p95_us':>8} {'min_us':>8} {'max_us':>8}  "
          f"grid (x,y,z)  kernel")
    for (name, gx, gy, gz), ns in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        ns = sorted(ns)
        p5, p95 = ns[int(round(0.05 * (len(ns) - 1)))], ns[int(round(0.95 * (len(ns) - 1)))]
        print(f"{len(ns):6d} {statistics.fmean(ns) / 1e3:9.3f} {p5 / 1e3:8.3f} {statistics.median(ns) / 1e3:9.3f} "
              f"{p95 / 1e3:8.3f} {ns[0] / 1e3:8.3f} {ns[-1] / 1e3:8.3f}  ({gx},{gy},{gz})  {name[:110]}")
    return 0


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gate_up_gemv_traffic.md")


def measured_traffic() -> dict | None:
    """HBM bytes per launch of the dominant kernel, from the two calibrated
    rocprofv3 --pmc passes recorded in the profile (a fenced json block)."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    if "```json" not in text:
        return None
    block = text.split("```json", 1)[1].split("```", 1)[0]
    return json.loads(block)


COPY_BYTES = 256 * 1024 * 1024


def main() -> int:
    args = parse()
    if args.trace_summary:
        return trace_summary(args.trace_summary)
    if args.phase_profile:
        # before anything imports the package: the ctypes binding loads this build
        os.environ.setdefault("TERNEL_TQ1_LIBRARY", os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                 "ternel_amd", "_lib", "libternel_tq1_profile.so"))
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the TQ1 path runs on a single MI355X in this build "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from ternel_amd import _lib, synthetic
    from ternel_amd.kernels import (GemmConfig, MatmulConfig, pack_weights, tq1_gemm_words, tq1_get_rows_words, tq1_linear_words,
                                    tq1_matmul_words, tq1_swiglu_words)
    from ternel_amd.layout import PackedTensorLayout
    from ternel_amd.modules import select_kernel

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    def events() -> tuple:
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def graph_of(fn):
        """Capture fn() into a HIP graph (after one eager call that sizes the workspace)."""
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        torch.cuda.synchronize()
        return graph

    def time_graph(graph, replays: int = 1) -> float:
        """ms per replay, events around the replays on the current stream."""
        stream = torch.cuda.current_stream(dev)
        a, b = events()
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(replays):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / replays

    if args.stream_ceiling:
        return stream_ceiling(torch, dev, graph_of, time_graph)
    if args.dense_reference:
        return dense_reference(torch, dev, graph_of, time_graph)
    if args.phase_profile:
        return phase_profile(torch, dev, synthetic, pack_weights, tq1_matmul_words, tq1_linear_words,
                             PackedTensorLayout, MatmulConfig, graph_of, time_graph, args.phase_batch)

    if args.prefill_probe:
        # Eager launches only (counter collection serialises dispatches).
        for name, K, N in C3_SHAPES:
            lay = PackedTensorLayout.for_tensor(N, K)
            blk = pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 3), layout=lay)
            xp = synthetic.device_activations(PREFILL_BATCHES[0], K, seed=synthetic.SEED_BASE + 3, sigma=0.5)
            for _ in range(2 + args.steps):
                tq1_gemm_words(blk, xp, layout=lay, config=GemmConfig())
            torch.cuda.synchronize()
            del blk, xp
        print(json.dumps({"prefill_probe": [name for name, _, _ in C3_SHAPES], "M": PREFILL_BATCHES[0],
                          "launches": 2 + args.steps}), flush=True)
        return 0

    # ---- config 1: ring of distinct weight copies, cold ----------------------------
    step_bytes = sum(packed_bytes(K, N) for _, K, N in C1_SHAPES)
    # One ring per matrix, each at least RING_BYTES_MIN and RING_COPIES_MIN
    # distinct copies: every cell that rotates one matrix reads it cold.
    rings = [ring_copies(packed_bytes(K, N)) for _, K, N in C1_SHAPES]
    ring_bytes = [r * packed_bytes(K, N) for r, (_, K, N) in zip(rings, C1_SHAPES)]
    layouts = [PackedTensorLayout.for_tensor(N, K) for _, K, N in C1_SHAPES]
    weights = [[pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 1 + 100 * r + i), layout=lay)
                for r in range(ring)] for i, ((_, K, N), lay, ring) in enumerate(zip(C1_SHAPES, layouts, rings))]
    ring = max(rings)  # steps of the three-matrix loop before every matrix has cycled its ring
    xs = [synthetic.device_activations(1, K, seed=synthetic.SEED_BASE + 1 + i) for i, (_, K, _) in enumerate(C1_SHAPES)]
    config = MatmulConfig()

    def step(r: int) -> None:
        for i, lay in enumerate(layouts):
            tq1_matmul_words(weights[i][r % rings[i]], xs[i], layout=lay, config=config)

    for w in range(args.warmup):
        step(w % ring)
    torch.cuda.synchronize()

    if args.traffic_probe:
        # Eager launches only (counter collection serialises dispatches): the dominant
        # kernel over the cold ring, then a plain copy of known size for calibration.
        xt = xs[0] if args.traffic_batch == 1 else synthetic.device_activations(
            args.traffic_batch, C1_SHAPES[0][1], seed=synthetic.SEED_BASE + 1)
        for s in range(args.steps):
            tq1_linear_words(weights[0][s % rings[0]], xt, layout=layouts[0])
        src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"traffic_probe": C1_SHAPES[0][0], "batch": args.traffic_batch, "launches": args.steps,
                          "bytes_per_launch": packed_bytes(C1_SHAPES[0][1], C1_SHAPES[0][2]),
                          "copy_bytes": COPY_BYTES}), flush=True)
        return 0

    # Timed region: exactly `steps` steps, replayed from one graph (no host
    # launch overhead between kernels), synchronize on both sides.
    steps_graph = graph_of(lambda: [step(s % ring) for s in range(args.steps)])
    ms_per_step = time_graph(steps_graph) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    del steps_graph

    # Dominant kernel (gate/up): `steps` cold launches back to back from one graph,
    # HIP events around them on the launch stream -> average launch duration.
    dominant = 0
    dom_name, dom_K, dom_N = C1_SHAPES[dominant]
    dom_bytes = packed_bytes(dom_K, dom_N)
    dom_graph = graph_of(lambda: [tq1_matmul_words(weights[dominant][s % rings[dominant]], xs[dominant], layout=layouts[dominant],
                                             config=config) for s in range(args.steps)])
    graph_launch_ms = time_graph(dom_graph) / args.steps
    del dom_graph
    achieved = dom_bytes / (graph_launch_ms * 1e-3) / 1e9
    # Eager launches bracketed one by one by event pairs (includes dispatch latency).
    stream = torch.cuda.current_stream(dev)
    pairs = [events() for _ in range(args.steps)]
    for s in range(args.steps):
        pairs[s][0].record(stream)
        tq1_matmul_words(weights[dominant][s % rings[dominant]], xs[dominant], layout=layouts[dominant], config=config)
        pairs[s][1].record(stream)
    torch.cuda.synchronize()
    launch_ms = sorted(a.elapsed_time(b) for a, b in pairs)
    mean_launch_ms = sum(launch_ms) / len(launch_ms)

    def quantile(q: float) -> float:  # nearest rank over the sorted launches
        return launch_ms[min(len(launch_ms) - 1, int(round(q * (len(launch_ms) - 1))))]
    per_matrix = {}
    for i, (name, K, N) in enumerate(C1_SHAPES):
        g = graph_of(lambda i=i: [tq1_matmul_words(weights[i][s % rings[i]], xs[i], layout=layouts[i], config=config)
                                  for s in range(rings[i] * 4)])
        ms = sorted(time_graph(g) for _ in range(3))[1] / (rings[i] * 4)  # median of three replays
        per_matrix[name] = {"graph_ms_per_launch": round(ms, 5), "GB/s": round(packed_bytes(K, N) / (ms * 1e-3) / 1e9, 1),
                            "ring_copies": rings[i], "ring_MiB": round(ring_bytes[i] / 2**20)}
        del g
    warm = graph_of(lambda: [tq1_matmul_words(weights[dominant][0], xs[dominant], layout=layouts[dominant], config=config)
                             for _ in range(100)])
    warm_ms = time_graph(warm) / 100
    del warm

    # ---- config 0: 4096 x 4096 at M=1, cold (a ring of distinct copies) and warm --
    c0_layout = PackedTensorLayout.for_tensor(C0_N, C0_K)
    c0_bytes = packed_bytes(C0_K, C0_N)
    c0_first = pack_weights(synthetic.device_blocks(C0_N, C0_K, seed=synthetic.SEED_BASE), layout=c0_layout)
    c0_ring = ring_copies(c0_bytes)
    c0_weights = [c0_first] + [c0_first.clone() for _ in range(c0_ring - 1)]
    c0_x = synthetic.device_activations(1, C0_K, seed=synthetic.SEED_BASE)
    config0 = {"workload": "BASELINE configs[0]: M=1, K=N=4096, fp16 activations, LUT23 GEMV "
                           "(the automatic configuration: the strip form)",
               "packed_bytes": c0_bytes, "kernel": select_kernel(c0_layout, 1, torch.float16),
               "form": m1_form(_lib.lib(), C0_N, C0_K)}
    for label, copies in (("cold", c0_ring), ("warm", 1)):
        launches = max(c0_ring, 200)
        g = graph_of(lambda copies=copies: [tq1_matmul_words(c0_weights[s % copies], c0_x, layout=c0_layout,
                                                             config=config) for s in range(launches)])
        ms = time_graph(g, 3) / launches  # time_graph gives ms per replay
        del g
        config0[label] = {"us": round(ms * 1e3, 3), "GB/s": round(c0_bytes / (ms * 1e-3) / 1e9, 1),
                          "copies": copies}
    config0["cold"]["note"] = f"{c0_ring} distinct copies ({c0_ring * c0_bytes >> 20} MiB) in rotation"
    config0["warm"]["note"] = "one copy, MALL/L2-resident after the first launch"
    del c0_weights, c0_first

    # ---- config 2: small batches over the same cold ring (library dispatch) ------
    small_batch = {}
    if not args.no_small_batch:
        for M in SMALL_BATCHES:
            xm = [synthetic.device_activations(M, K, seed=synthetic.SEED_BASE + 2 + M) for _, K, _ in C1_SHAPES]
            row = {}
            for i, (name, K, N) in enumerate(C1_SHAPES):
                g = graph_of(lambda i=i: [tq1_linear_words(weights[i][s % rings[i]], xm[i], layout=layouts[i])
                                          for s in range(rings[i] * 2)])
                ms = sorted(time_graph(g) for _ in range(3))[1] / (rings[i] * 2)  # median of three replays
                del g
                row[name] = {"us": round(ms * 1e3, 2),
                             "GB/s": round(packed_bytes(K, N) / (ms * 1e-3) / 1e9, 1),
                             "TFLOP/s": round(2 * M * K * N / (ms * 1e-3) / 1e12, 2),
                             "kernel": select_kernel(layouts[i], M, torch.float16)}
            small_batch[f"M={M}"] = row
            del xm
    traffic = measured_traffic()

    result = {
        "metric": "packed-weight GB/s at M=1 (TQ1_G128 decode GEMV, 27B-class shapes)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "activation_dtype": "f16",
        "data": "synthetic (BASELINE trit/scale/activation distributions; one cold ring per matrix of "
                f"{'/'.join(str(r) for r in rings)} distinct copies, "
                f"{'/'.join(str(round(b / 2**20)) for b in ring_bytes)} MiB); steps replayed from a HIP graph",
        "config": {
            "workload": "BASELINE configs[1]: M=1 GEMV over gate/up 5120->17408, down 17408->5120, "
                        "QKV 5120->8192 (one step = the three GEMVs)",
            "M": 1,
            "packed_bytes_per_step": step_bytes,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "per_matrix": per_matrix,
        "warm_gate_up_GBs": round(dom_bytes / (warm_ms * 1e-3) / 1e9, 1),
        "config0": config0,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes_per_launch"] if traffic else None,
            "kernel": f"{dom_name} GEMV K={dom_K} N={dom_N} ("
                      + {"strip": "strip_gemv_kernel: every row reduced inside one workgroup, no split",
                         "lut23": "lut_gemv_kernel, fused ordered split-K"}.get(
                          m1_form(_lib.lib(), dom_N, dom_K),
                          "strip_gemv_kernel in K chunks meeting in exchange slots") + ")",
            "bytes_per_launch": dom_bytes,
            "mean_launch_us": round(graph_launch_ms * 1e3, 3),
            "timing": f"{args.steps} cold launches back to back in one HIP graph, events on the launch stream",
            "eager_event_pair_mean_us": round(mean_launch_ms * 1e3, 3),
            "eager_event_pair_us": {"p5": round(quantile(0.05) * 1e3, 3), "median": round(quantile(0.5) * 1e3, 3),
                                    "p95": round(quantile(0.95) * 1e3, 3), "launches": len(launch_ms),
                                    "timing": "one event pair around each eager launch (dispatch included), "
                                              "as the reference's per-launch statistics"},
            "traffic_detail": traffic,
        },
    }
    if small_batch:
        result["small_batch"] = {"workload": "BASELINE configs[2]: M in {2..64} over the three configs[1] "
                                             "matrices, cold ring, library dispatch (ternel_tq1_linear)",
                                 **small_batch}
    del weights

    # ---- config 3: prefill GEMM M=512 and M=2048 ---------------------------------
    if not args.no_prefill:
        for M in PREFILL_BATCHES:
            prefill = {}
            for name, K, N in C3_SHAPES:
                lay = PackedTensorLayout.for_tensor(N, K)
                blk = pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 3), layout=lay)
                xp = synthetic.device_activations(M, K, seed=synthetic.SEED_BASE + 3, sigma=0.5)
                reps = max(4, 20 * 512 // M)
                g = graph_of(lambda: [tq1_gemm_words(blk, xp, layout=lay, config=GemmConfig()) for _ in range(reps)])
                ms = time_graph(g) / reps
                tflops = 2 * M * K * N / (ms * 1e-3) / 1e12
                prefill[name] = {"ms": round(ms, 4), "TFLOP/s": round(tflops, 2),
                                 "frac_of_mfma_f16_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
                del g, blk, xp
            result[f"prefill_m{M}"] = prefill
        # bf16 activations at M=512: the wide form after the per-row power-of-two
        # conversion to fp16 (exact), fp32 sums rounded once to bf16
        M = PREFILL_BATCHES[0]
        prefill = {}
        for name, K, N in C3_SHAPES:
            lay = PackedTensorLayout.for_tensor(N, K)
            blk = pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 3), layout=lay)
            xp = synthetic.device_activations(M, K, seed=synthetic.SEED_BASE + 3, sigma=0.5).to(torch.bfloat16)
            g = graph_of(lambda: [tq1_gemm_words(blk, xp, layout=lay, config=GemmConfig()) for _ in range(20)])
            ms = time_graph(g) / 20
            tflops = 2 * M * K * N / (ms * 1e-3) / 1e12
            fp16_ms = result[f"prefill_m{M}"][name]["ms"]
            prefill[name] = {"ms": round(ms, 4), "TFLOP/s": round(tflops, 2),
                             "frac_of_mfma_f16_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                             "vs_fp16": round(ms / fp16_ms, 3)}
            del g, blk, xp
        result[f"prefill_m{M}_bf16"] = prefill

    # ---- the tied output head at M=1 (scope row f3): the largest GEMV of a token --
    if not args.no_model_stream:
        head_layout = PackedTensorLayout.for_tensor(HEAD_ROWS, 5120)
        heads = [pack_weights(synthetic.device_blocks(HEAD_ROWS, 5120, seed=synthetic.SEED_BASE + 50 + i),
                              layout=head_layout) for i in range(2)]  # 2 x 278 MB: every launch reads HBM
        xh = synthetic.device_activations(1, 5120, seed=synthetic.SEED_BASE + 51)
        g = graph_of(lambda: [tq1_matmul_words(heads[s % 2], xh, layout=head_layout, config=MatmulConfig())
                              for s in range(20)])
        ms = time_graph(g) / 20
        head_bytes = packed_bytes(5120, HEAD_ROWS)
        result["head_m1"] = {"workload": f"tied output head {HEAD_ROWS}x5120 at M=1 (PackedEmbedding.as_linear, "
                                         "two alternating copies)",
                             "us": round(ms * 1e3, 2), "GB/s": round(head_bytes / (ms * 1e-3) / 1e9, 1),
                             "frac_of_hbm_peak": round(head_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del g, heads

    # ---- config 4: 64-layer weight stream + one embedding row -------------------
    if not args.no_model_stream:
        result["model_stream"] = model_stream(torch, synthetic, pack_weights, tq1_matmul_words, tq1_get_rows_words, tq1_swiglu_words,
                                              PackedTensorLayout, MatmulConfig, graph_of, time_graph)
        result["census_stream"] = census_stream(torch, synthetic, pack_weights, PackedTensorLayout, graph_of, time_graph)

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)

    print(json.dumps(result), flush=True)
    return 0


PHASES = ("start", "activations arrived", "first words issued", "own tables written", "tables ready (barrier)",
          "blocks summed", "partial stored and acknowledged", "arrival counted", "fix-up done")
# The strip GEMV's stamps (M=1 where a CU's strip is at most 96 rows: gate/up, QKV, and down in
# four K chunks, whose `done` includes the chunks' exchange).
STRIP_PHASES = ("start", "activations arrived, first words issued", "tables ready", "all items summed", "done")
# The wide form's stamps in the same slots (2-4 unused; 7 and 8 only where it reduces a shared tile).
WIDE_PHASES = ("start", "first unit's operands in LDS", "-", "-", "-", "segment summed", "arrival counted",
               "other contributors' partials published", "tile stored")


def phase_profile(torch, dev, synthetic, pack_weights, tq1_matmul_words, tq1_linear_words, PackedTensorLayout,
                  MatmulConfig, graph_of, time_graph, batch: int = 1) -> int:
    """Per configs[1] matrix: three cold launches of the M=1 GEMV (the LUT23
    kernel; with batch > 1 the kernel the library's dispatch picks, of which
    the direct-fragment and wide forms are stamped, the wide form with its own
    phase names) with the phase stamps of every wave
    (100 MHz wall clock, lane 0) and the XCC it ran on. Wall clocks of different XCCs are not comparable,
    so every time is taken against the first wave start of the wave's own
    XCC: each phase's time, the XCC's span (first start to last stamp), each
    phase's duration per wave, and the time to the tables by the quarter of
    the XCC's waves a wave started in; beside them the graph-timed GEMV of
    the same build over a cold ring."""
    import ctypes
    import statistics

    from ternel_amd import _lib

    handle = _lib.lib()
    fn = handle.ternel_tq1_profile_stamps
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    max_waves = 8192
    slots = 16  # the phases, then (last slot) 1 + the XCC id
    buf = (ctypes.c_ulonglong * (max_waves * slots))()

    def quantiles(values: list) -> dict:
        values = sorted(values)
        return {"median_us": round(statistics.median(values), 2),
                "p95_us": round(values[int(0.95 * (len(values) - 1))], 2), "max_us": round(values[-1], 2)}

    for i, (name, K, N) in enumerate(C1_SHAPES):
        wide = batch > 1 and handle.ternel_tq1_linear_kernel(batch, N, K, 0) == 3  # TERNEL_TQ1_GEMM_WIDE
        strip = batch == 1 and m1_form(handle, N, K).startswith("strip")
        lut = handle.ternel_tq1_linear_kernel(batch, N, K, 0) == 100  # TERNEL_TQ1_KERNEL_LUT23
        names = WIDE_PHASES if wide else (STRIP_PHASES if strip else PHASES)
        lay = PackedTensorLayout.for_tensor(N, K)
        ring = ring_copies(packed_bytes(K, N))
        weights = [pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 1 + 100 * r + i), layout=lay)
                   for r in range(ring)]
        x = synthetic.device_activations(batch, K, seed=synthetic.SEED_BASE + 1 + i)

        def gemv(w):
            return tq1_matmul_words(w, x, layout=lay) if batch == 1 else tq1_linear_words(w, x, layout=lay)

        graph_ms = time_graph(graph_of(lambda: [gemv(weights[r % ring]) for r in range(ring * 4)])) / (ring * 4)
        phase_times = {phase: [] for phase in names if phase != "-"}
        spans, durations, by_start = [], {}, [[] for _ in range(4)]
        for r in range(3):  # three cold launches, each over a copy not read for ring - 1 launches
            fn(buf, max_waves, torch.cuda.current_stream(dev).cuda_stream)
            gemv(weights[(r + 5) % ring])
            waves = fn(buf, max_waves, torch.cuda.current_stream(dev).cuda_stream)
            stamps = [[buf[w * slots + p] for p in range(slots)] for w in range(waves)]
            stamps = [st for st in stamps if st[0] and st[slots - 1]]
            for xcc in {st[slots - 1] for st in stamps}:
                mine = [st for st in stamps if st[slots - 1] == xcc]
                t0 = min(st[0] for st in mine)
                spans.append(max(max(v for v in st[:len(names)] if v) for st in mine) / 100 - t0 / 100)
                for p, phase in enumerate(names):
                    if phase != "-":
                        phase_times[phase] += [(st[p] - t0) / 100 for st in mine if st[p]]
                ranked = sorted(mine, key=lambda st: st[0])
                quarter = max(1, len(ranked) // 4)
                for q in range(4 if names is PHASES else 0):
                    part = ranked[q * quarter:(q + 1) * quarter] if q < 3 else ranked[3 * quarter:]
                    by_start[q] += [((st[0] - t0) / 100, (st[3] - st[0]) / 100, (st[1] - st[0]) / 100,
                                     (st[2] - st[1]) / 100) for st in part if st[3] and st[1] and st[2]]
            for st in stamps:  # between consecutive phases the wave stamped
                present = [p for p in range(len(names)) if st[p]]
                for a, b in zip(present, present[1:]):
                    durations.setdefault(f"{names[a]} -> {names[b]}", []).append((st[b] - st[a]) / 100)
        if not spans:  # the dispatch picked a kernel without phase stamps (the tile form)
            print(json.dumps({"phase_profile": name, "K": K, "N": N, "M": batch,
                              "kernel": handle.ternel_tq1_linear_kernel(batch, N, K, 0),
                              "note": "no phase stamps: the kernel the dispatch picks here is not stamped"}),
                  flush=True)
            del weights
            continue
        print(json.dumps({
            "phase_profile": name, "K": K, "N": N, "M": batch, "waves_per_launch": len(phase_times["start"]) // 3,
            "kernel": "wide_gemm_kernel" if wide else (f"strip_gemv_kernel ({m1_form(handle, N, K)})" if strip else
                                                        ("lut_gemv_kernel" if lut else "direct_gemm_kernel")),
            "gemv_graph_us": round(graph_ms * 1e3, 3),
            "xcc_span_us": quantiles(spans),
            "phases_after_xcc_first_wave_start": {ph: quantiles(v) for ph, v in phase_times.items() if v},
            "phase_durations_per_wave": {k: quantiles(v) for k, v in durations.items() if v},
            "tables_by_start_quarter": [
                {"started_after_xcc_first_us": round(statistics.median(v[0] for v in part), 2),
                 "start_to_tables_written_us": round(statistics.median(v[1] for v in part), 2),
                 "start_to_activations_us": round(statistics.median(v[2] for v in part), 2),
                 "activations_to_words_issued_us": round(statistics.median(v[3] for v in part), 2)}
                for part in by_start if part],
            "clock": "s_memrealtime (100 MHz), lane 0 of every wave, grouped by HW_REG_XCC_ID, 3 cold launches"}),
            flush=True)
        del weights
    return 0


DENSE_BATCHES = (1, 16, 512, 2048)


def dense_reference(torch, dev, graph_of, time_graph) -> int:
    """The same products with dense fp16 weights through torch.mm (hipBLASLt / rocBLAS):
    what a vendor-library GEMM of the unpacked matrix costs on this GPU. y = x @ Wt with
    Wt a contiguous (K, N) fp16 matrix (2 bytes per weight against the packed 0.219).
    Batches up to 16 rotate over a ring of distinct weight copies (cold, HBM-bound);
    512 and 2048 reuse one copy (MFMA-bound, the weight read is 3-10 % of the time).
    Eager launches back to back between one event pair (a library call is not put into
    a graph here: it may record memset nodes)."""
    del graph_of, time_graph

    def timed(fn, launches: int) -> float:
        fn(0)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for s in range(launches):
            fn(s)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / launches * 1e3

    for name, K, N in C1_SHAPES:
        dense_bytes = K * N * 2
        ring = max(2, -(-RING_BYTES_MIN // dense_bytes))
        gen = torch.Generator(device=dev).manual_seed(2024)
        weights = [(torch.randn(K, N, device=dev, generator=gen) * 0.02).half() for _ in range(ring)]
        for M in DENSE_BATCHES:
            x = torch.randn(M, K, device=dev, generator=gen).half()
            copies = ring if M <= 16 else 1
            launches = ring * 4 if M <= 16 else 20
            us = sorted(timed(lambda s: torch.mm(x, weights[s % copies]), launches) for _ in range(3))[1]
            flops = 2.0 * M * K * N
            print(json.dumps({"dense_reference": name, "K": K, "N": N, "M": M, "dtype": "f16",
                              "weights": "cold ring" if copies > 1 else "one copy", "us": round(us, 2),
                              "TFLOP/s": round(flops / us / 1e6, 1),
                              "weight_GB/s": round(dense_bytes / us / 1e3, 1),
                              "packed_bytes": packed_bytes(K, N), "dense_bytes": dense_bytes}), flush=True)
        del weights
        torch.cuda.empty_cache()
    return 0


STREAM_SIZES = (("qkv", 9_175_040), ("gate_up", 19_496_960), ("layer", 76_840_960), ("long", 320 * 2**20))
# (load width in bytes, loads per lane, threads per workgroup)
STREAM_SHAPES = ((4, 7, 512), (4, 28, 256), (16, 2, 512), (16, 4, 512), (16, 8, 256), (16, 16, 256))
STREAM_POOL_BYTES = 1536 * 2**20  # rotation pool: every launch reads bytes no cache holds


def stream_ceiling(torch, dev, graph_of, time_graph) -> int:
    """Single-launch read ceiling: for each matrix size and load shape, 64 launches replayed
    from one graph, each over a different region of a 1.5 GiB pool (cold), of a kernel that
    only loads (every load issued before the first use) and writes one word per wave."""
    import ctypes

    from ternel_amd.build import PROBE_PATH

    if not PROBE_PATH.exists():
        raise RuntimeError(f"{PROBE_PATH} is missing; build with `python -m ternel_amd.build`")
    probe = ctypes.CDLL(str(PROBE_PATH))
    probe.ternel_probe_chunk_bytes.restype = ctypes.c_int64
    probe.ternel_probe_chunk_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    probe.ternel_probe_stream.restype = ctypes.c_int
    probe.ternel_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    probe.ternel_probe_last_error.restype = ctypes.c_char_p
    pool = torch.ones(STREAM_POOL_BYTES // 4, dtype=torch.int32, device=dev)
    max_waves = max(size // probe.ternel_probe_chunk_bytes(w, l) for _, size in STREAM_SIZES
                    for w, l, _ in STREAM_SHAPES)
    out = torch.zeros(max_waves, dtype=torch.int32, device=dev)
    launches = 64
    rows = []
    for name, size in STREAM_SIZES:
        for width, loads, threads in STREAM_SHAPES:
            chunk = probe.ternel_probe_chunk_bytes(width, loads)
            waves = size // chunk
            nbytes = waves * chunk
            stride = -(-nbytes // 4096) * 4096
            regions = min(launches, STREAM_POOL_BYTES // stride)

            def launch(r, waves=waves, width=width, loads=loads, threads=threads, stride=stride, regions=regions):
                offset = (r % regions) * stride
                rc = probe.ternel_probe_stream(pool.data_ptr() + offset, STREAM_POOL_BYTES - offset, out.data_ptr(),
                                               out.numel(), waves, width, loads, threads,
                                               torch.cuda.current_stream(dev).cuda_stream)
                if rc != 0:
                    raise RuntimeError(probe.ternel_probe_last_error().decode())

            g = graph_of(lambda: [launch(r) for r in range(launches)])
            ms = min(time_graph(g) for _ in range(3)) / launches
            del g
            rows.append({"size": name, "bytes": nbytes, "width": width, "loads_per_lane": loads,
                         "threads": threads, "workgroups": -(-waves // (threads // 64)), "regions": regions,
                         "us": round(ms * 1e3, 3), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)})
            print(json.dumps(rows[-1]), flush=True)
    best = {}
    for row in rows:
        if row["size"] not in best or row["GB/s"] > best[row["size"]]["GB/s"]:
            best[row["size"]] = row
    print(json.dumps({"stream_ceiling": {k: {"us": v["us"], "GB/s": v["GB/s"],
                                            "frac_of_hbm_peak": round(v["GB/s"] / HBM_PEAK_GBS, 4),
                                            "shape": [v["width"], v["loads_per_lane"], v["threads"]]}
                                        for k, v in best.items()},
                      "timing": f"{launches} launches per graph over distinct pool regions, best of 3 replays"}),
          flush=True)
    return 0


C4_LAYER = (("qkv", 5120, 8192), ("o", 8192, 5120), ("gate_up", 5120, 34816), ("down", 17408, 5120))
C4_LAYERS = 64
C4_VOCAB = 151936
PREFILL_TOKENS = 8192
HEAD_ROWS = 248320  # Bonsai 27B vocabulary: the tied lm_head (src/ternel_mlx/layout.py:179-192 census)


def model_stream(torch, synthetic, pack_weights, tq1_matmul_words, tq1_get_rows_words, tq1_swiglu_words, PackedTensorLayout,
                 MatmulConfig, graph_of, time_graph) -> dict:
    """64 sequential layers of M=1 GEMVs (4.92 GB of packed weights,
    larger than every cache, so each token reads them cold), then one embedding row. The
    gate+up weight (its rows alternating gate, up) runs as the fused SwiGLU, so each layer
    also produces the MLP's activation; the packed bytes are the same."""
    layouts = [PackedTensorLayout.for_tensor(N, K) for _, K, N in C4_LAYER]
    weights = [[pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 4 + 10 * layer + i), layout=lay)
                for i, ((_, K, N), lay) in enumerate(zip(C4_LAYER, layouts))] for layer in range(C4_LAYERS)]
    xs = {K: synthetic.device_activations(1, K, seed=synthetic.SEED_BASE + 4 + K) for _, K, _ in C4_LAYER}
    table_layout = PackedTensorLayout.for_tensor(C4_VOCAB, 5120)
    table = pack_weights(synthetic.device_blocks(C4_VOCAB, 5120, seed=synthetic.SEED_BASE + 44), layout=table_layout)
    token = torch.tensor([75967], dtype=torch.int64, device="cuda")
    config = MatmulConfig()

    def token_pass() -> None:
        for layer in range(C4_LAYERS):
            for i, (name, K, _) in enumerate(C4_LAYER):
                if name == "gate_up":
                    tq1_swiglu_words(weights[layer][i], xs[K], layout=layouts[i])
                else:
                    tq1_matmul_words(weights[layer][i], xs[K], layout=layouts[i], config=config)
        tq1_get_rows_words(table, token, layout=table_layout, dtype=torch.float16)

    graph = graph_of(token_pass)
    replays = 5
    ms = time_graph(graph, replays)
    total = C4_LAYERS * sum(packed_bytes(K, N) for _, K, N in C4_LAYER)
    gather = graph_of(lambda: [tq1_get_rows_words(table, token, layout=table_layout, dtype=torch.float16) for _ in range(100)])
    gather_us = time_graph(gather) / 100 * 1e3
    # A prefill's gather: 8192 random ids, 1120 packed bytes read and 10240 fp16 bytes
    # written per row, HBM-bound on the writes.
    ids = torch.randint(0, C4_VOCAB, (PREFILL_TOKENS,), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(synthetic.SEED_BASE + 45))
    prefill_bytes = PREFILL_TOKENS * (packed_bytes(5120, 1) + 5120 * 2)
    # PackedEmbedding gathers from its canonical row-major copy (a token's 1120 bytes
    # contiguous); the packed layout spreads a row over 280 separate 256-byte segments.
    from ternel_amd.kernels import tq1_get_rows_canonical, unpack_weights
    rows_major = unpack_weights(table, layout=table_layout)
    prefill = graph_of(lambda: [tq1_get_rows_canonical(rows_major, ids, layout=table_layout, dtype=torch.float16)
                                for _ in range(10)])
    prefill_us = time_graph(prefill, 5) / 10 * 1e3
    from_packed = graph_of(lambda: [tq1_get_rows_words(table, ids, layout=table_layout, dtype=torch.float16)
                                    for _ in range(10)])
    from_packed_us = time_graph(from_packed, 5) / 10 * 1e3
    del graph, gather, prefill, from_packed, weights, table, rows_major
    return {
        "workload": "BASELINE configs[4]: 64 x (QKV 5120->8192, O 8192->5120, gate+up 5120->34816 with the "
                    "fused SwiGLU epilogue, down 17408->5120) M=1 GEMVs + 1 embedding row of 151936x5120, "
                    "one HIP graph per token",
        "packed_bytes": total,
        "ms_per_token": round(ms, 4),
        "GB/s": round(total / (ms * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "embedding_row_us_graph": round(gather_us, 3),
        "embedding_prefill": {"tokens": PREFILL_TOKENS, "table": "canonical rows (PackedEmbedding)",
                              "us": round(prefill_us, 2), "bytes": prefill_bytes,
                              "GB/s": round(prefill_bytes / prefill_us / 1e3, 1),
                              "frac_of_hbm_peak": round(prefill_bytes / prefill_us / 1e3 / HBM_PEAK_GBS, 4),
                              "packed_table_us": round(from_packed_us, 2)},
    }


FULL_ATTENTION_INTERVAL = 4  # every fourth layer is full attention (the reference's tests/test_mlx_modules.py:71)


def census_order() -> list:
    """The 497 linear tensors of one decoded token in model order: 64 layers, a
    full-attention layer (q, k, v, o) every fourth and linear attention (qkv,
    z, a, b, out) in the others, each with its MLP (gate, up, down), then the
    tied head -- the census of src/ternel_mlx/layout.py:179-195, whose
    per-shape counts this order reproduces (checked below)."""
    from ternel_amd.layout import DISPATCHES_PER_TOKEN, MODEL_LINEAR_SHAPES
    order = []
    for layer in range(C4_LAYERS):
        if layer % FULL_ATTENTION_INTERVAL == FULL_ATTENTION_INTERVAL - 1:
            order += [("self_attn.q_proj", 12288, 5120), ("self_attn.k_proj", 1024, 5120),
                      ("self_attn.v_proj", 1024, 5120), ("self_attn.o_proj", 5120, 6144)]
        else:
            order += [("linear_attn.in_proj_qkv", 10240, 5120), ("linear_attn.in_proj_z", 6144, 5120),
                      ("linear_attn.in_proj_a", 48, 5120), ("linear_attn.in_proj_b", 48, 5120),
                      ("linear_attn.out_proj", 5120, 6144)]
        order += [("mlp.gate_proj", 17408, 5120), ("mlp.up_proj", 17408, 5120), ("mlp.down_proj", 5120, 17408)]
    order.append(("lm_head", HEAD_ROWS, 5120))
    counts = {}
    for _, rows, columns in order:
        counts[(rows, columns)] = counts.get((rows, columns), 0) + 1
    census = {(s.rows, s.columns): s.dispatches_per_token for s in MODEL_LINEAR_SHAPES}
    if len(order) != DISPATCHES_PER_TOKEN or counts != census:
        raise RuntimeError("the model order does not reproduce the 27B shape census")
    return order


def census_stream(torch, synthetic, pack_weights, PackedTensorLayout, graph_of, time_graph) -> dict:
    """The reference's whole-model traversal (reports_v2/03_streaming_benchmark.md:5,10: 497 tensors,
    5,604,802,560 packed bytes, 11.273 ms = 497.181 GB/s): every tensor once, in model order, as an
    M=1 GEMV through the library's automatic configuration, each a distinct weight (5.6 GB, larger
    than every cache). Each GEMV reads the previous one's output: two fp16 buffers alternate as
    input and output (a GEMV with fewer outputs than the next one's columns leaves the rest of its
    output buffer from earlier GEMVs), so no launch can start before the one it follows ends. One
    HIP graph per traversal. Then every shape alone: its copies of the traversal in rotation."""
    from ternel_amd import _lib
    from ternel_amd.kernels import workspace
    order = census_order()
    handle = _lib.lib()
    lays = [PackedTensorLayout.for_tensor(rows, columns) for _, rows, columns in order]
    weights = [pack_weights(synthetic.device_blocks(rows, columns, seed=synthetic.SEED_BASE + 60 + i), layout=lay)
               for i, ((_, rows, columns), lay) in enumerate(zip(order, lays))]
    total = sum(packed_bytes(columns, rows) for _, rows, columns in order)
    width = max(max(rows, columns) for _, rows, columns in order)
    bufs = [synthetic.device_activations(1, width, seed=synthetic.SEED_BASE + 61 + i) for i in range(2)]
    need = max(handle.ternel_tq1_matmul_workspace_bytes(1, rows, columns, 0, 0) for _, rows, columns in order)
    ws = workspace(bufs[0].device, need)
    ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)

    def gemv(i: int, src, dst) -> None:
        _, rows, columns = order[i]
        _lib.check(handle.ternel_tq1_matmul(weights[i].data_ptr(), src.data_ptr(), dst.data_ptr(), 1, rows, columns,
                                            _lib.DTYPE_F16, 0, 0, ws_ptr, ws_bytes,
                                            torch.cuda.current_stream().cuda_stream))

    def traversal() -> None:
        for i in range(len(order)):
            gemv(i, bufs[i % 2], bufs[(i + 1) % 2])

    graph = graph_of(traversal)
    time_graph(graph)  # a full warm-up traversal (the reference runs six)
    ms = sorted(time_graph(graph) for _ in range(5))[2]  # median of five traversals
    del graph
    shapes = {}
    for name, rows, columns in order:
        key = f"{rows}x{columns}"
        if key in shapes:
            continue
        idx = [i for i, (_, r, c) in enumerate(order) if (r, c) == (rows, columns)]
        launches = max(len(idx), 16) if len(idx) > 1 else 8
        g = graph_of(lambda idx=idx, launches=launches: [gemv(idx[s % len(idx)], bufs[0], bufs[1])
                                                         for s in range(launches)])
        us = sorted(time_graph(g) for _ in range(3))[1] / launches * 1e3
        del g
        nbytes = packed_bytes(columns, rows)
        shapes[key] = {"tensor": name, "per_token": len(idx), "distinct_copies": len(idx), "us": round(us, 3),
                       "GB/s": round(nbytes / us / 1e3, 1), "kernel": m1_form(handle, rows, columns)}
    del weights, bufs
    return {
        "workload": "the reference's 497-tensor model-order traversal (27B census, src/ternel_mlx/layout.py:179-195): "
                    "M=1 GEMVs, each reading the previous one's output, one HIP graph per traversal",
        "tensors": len(order),
        "packed_bytes": total,
        "ms_per_traversal": round(ms, 4),
        "GB/s": round(total / (ms * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "reference_GBs": 497.181,
        "per_shape": shapes,
    }


if __name__ == "__main__":
    sys.exit(main())
