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
duration, from per-launch HIP event pairs recorded on the launch stream inside
the same timed region. The M=512 prefill GEMM is reported as a
secondary figure in TFLOP/s against the fp16 MFMA peak, and the reference's
CPU decode+matmul path (the oracle restatement) is timed on the host cores on a
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

C1_SHAPES = (("gate_up", 5120, 17408), ("down", 17408, 5120), ("qkv", 5120, 8192))  # (name, K, N)
C3_SHAPES = (("gate_up", 5120, 17408), ("down", 17408, 5120))
RING_BYTES_MIN = 600 * 1024 * 1024  # > 2 x (256 MiB MALL + L2)


def packed_bytes(K: int, N: int) -> int:
    return N * (K // 128) * 28


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
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


def cpu_baseline(seconds: float) -> dict:
    """The reference's CPU path (decode_tq1_blocks + numpy matmul), restated in the
    oracle, timed on a bounded sample: whole gate/up matrix decodes + matvecs."""
    import numpy as np

    from oracle import tq1_oracle as O
    from ternel_amd import synthetic

    name, K, N = C1_SHAPES[0]
    blocks = synthetic.host_blocks(N, K, seed=synthetic.SEED_BASE + 1)
    x = synthetic.host_activations(1, K, seed=synthetic.SEED_BASE + 1)
    calls = 0
    start = time.perf_counter()
    while True:
        O.cpu_decode_matmul(blocks, x, rows=N, columns=K)
        calls += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds:
            break
    per_call = elapsed / calls
    return {
        "value": round(packed_bytes(K, N) / per_call / 1e9, 4),
        "unit": "GB/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": (f"{calls} x full decode (oracle decode_tq1_blocks restatement) + fp32 numpy matvec of the "
                   f"{name} matrix K={K} N={N} ({packed_bytes(K, N)} packed bytes), {elapsed:.1f} s; "
                   f"decode is single-threaded numpy, the matvec uses the BLAS threads"),
        "seconds_per_call": round(per_call, 4),
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the TQ1 path runs on a single MI355X in this build "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from ternel_amd import synthetic
    from ternel_amd.kernels import GemmConfig, MatmulConfig, pack_weights, tq1_gemm, tq1_matmul
    from ternel_amd.layout import PackedTensorLayout

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    # ---- config 1: ring of distinct weight copies --------------------------------
    step_bytes = sum(packed_bytes(K, N) for _, K, N in C1_SHAPES)
    ring = max(2, -(-RING_BYTES_MIN // step_bytes))
    layouts = [PackedTensorLayout.for_tensor(N, K) for _, K, N in C1_SHAPES]
    weights = [[pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 1 + 100 * r + i), layout=lay)
                for i, ((_, K, N), lay) in enumerate(zip(C1_SHAPES, layouts))] for r in range(ring)]
    xs = [synthetic.device_activations(1, K, seed=synthetic.SEED_BASE + 1 + i) for i, (_, K, _) in enumerate(C1_SHAPES)]
    config = MatmulConfig()

    def step(r: int, starts=None, ends=None) -> None:
        for i, lay in enumerate(layouts):
            if starts is not None:
                starts[i].record(stream)
            tq1_matmul(weights[r][i], xs[i], layout=lay, config=config)
            if ends is not None:
                ends[i].record(stream)

    for w in range(args.warmup):
        step(w % ring)
    torch.cuda.synchronize()

    starts = [[torch.cuda.Event(enable_timing=True) for _ in C1_SHAPES] for _ in range(args.steps)]
    ends = [[torch.cuda.Event(enable_timing=True) for _ in C1_SHAPES] for _ in range(args.steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for s in range(args.steps):
        step(s % ring, starts[s], ends[s])
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps
    per_kernel_ms = [sum(starts[s][i].elapsed_time(ends[s][i]) for s in range(args.steps)) / args.steps
                     for i in range(len(C1_SHAPES))]
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    dominant = 0  # gate/up: the largest packed matrix, first in the step
    dom_bytes = packed_bytes(C1_SHAPES[dominant][1], C1_SHAPES[dominant][2])
    achieved = dom_bytes / (per_kernel_ms[dominant] * 1e-3) / 1e9

    # Warm (weights resident in MALL/L2) for context.
    warm_iters = 100
    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    tq1_matmul(weights[0][0], xs[0], layout=layouts[0], config=config)
    w0.record(stream)
    for _ in range(warm_iters):
        tq1_matmul(weights[0][0], xs[0], layout=layouts[0], config=config)
    w1.record(stream)
    torch.cuda.synchronize()
    warm_ms = w0.elapsed_time(w1) / warm_iters

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
        "data": "synthetic (BASELINE trit/scale/activation distributions; cold ring of "
                f"{ring} distinct weight copies, {ring * step_bytes / 2**20:.0f} MiB)",
        "config": {
            "workload": "BASELINE configs[1]: M=1 GEMV over gate/up 5120->17408, down 17408->5120, "
                        "QKV 5120->8192 (one step = the three GEMVs)",
            "M": 1,
            "packed_bytes_per_step": step_bytes,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "per_matrix": {name: {"ms": round(ms, 5), "GB/s": round(packed_bytes(K, N) / (ms * 1e-3) / 1e9, 1)}
                       for (name, K, N), ms in zip(C1_SHAPES, per_kernel_ms)},
        "warm_gate_up_GBs": round(dom_bytes / (warm_ms * 1e-3) / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "gate/up GEMV 5120->17408 (lut_gemv_kernel, fused ordered split-K)",
            "bytes_per_launch": dom_bytes,
        },
    }

    # ---- config 3: prefill GEMM M=512 ------------------------------------------
    if not args.no_prefill:
        prefill = {}
        for name, K, N in C3_SHAPES:
            lay = PackedTensorLayout.for_tensor(N, K)
            blk = pack_weights(synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 3), layout=lay)
            xp = synthetic.device_activations(512, K, seed=synthetic.SEED_BASE + 3, sigma=0.5)
            for _ in range(3):
                tq1_gemm(blk, xp, layout=lay, config=GemmConfig())
            p0 = torch.cuda.Event(enable_timing=True)
            p1 = torch.cuda.Event(enable_timing=True)
            iters = 20
            p0.record(stream)
            for _ in range(iters):
                tq1_gemm(blk, xp, layout=lay, config=GemmConfig())
            p1.record(stream)
            torch.cuda.synchronize()
            ms = p0.elapsed_time(p1) / iters
            tflops = 2 * 512 * K * N / (ms * 1e-3) / 1e12
            prefill[name] = {"ms": round(ms, 4), "TFLOP/s": round(tflops, 2),
                             "frac_of_mfma_f16_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
            del blk, xp
        result["prefill_m512"] = prefill

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
