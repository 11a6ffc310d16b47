"""Dispatch sweep on an MI355X: every kernel the library can run for each
(shape, batch) of the 27B linears, timed the way bench.py times (cold weight
ring, launches replayed from one HIP graph). Writes the fixture that
tests/test_dispatch.py replays through the library's own dispatch rule, as the
reference replays its sweeps through select_gemm (tests/test_mlx_modules.py
:553,1007).

    python tests/golden/sweep_dispatch.py OUT.json     # on a GPU box
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from ternel_amd import synthetic  # noqa: E402
from ternel_amd.kernels import GemmConfig, MatmulConfig, pack_weights, tq1_gemm_words, tq1_matmul_words  # noqa: E402
from ternel_amd.layout import PackedTensorLayout  # noqa: E402

SHAPES = (("gate_up", 5120, 17408), ("down", 17408, 5120), ("qkv", 5120, 8192), ("o", 8192, 5120))
BATCHES = (1, 2, 3, 4, 5, 6, 8, 12, 16, 24, 32, 40, 48, 64, 96, 128, 256, 512)
RING_BYTES = 700 << 20


def graph_us(fn, launches: int) -> float:
    fn(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(launches):
            fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / launches * 1e3


def main(out: str) -> None:
    rows = []
    for name, K, N in SHAPES:
        lay = PackedTensorLayout.for_tensor(N, K)
        ring = max(2, RING_BYTES // lay.payload_bytes)
        weights = [pack_weights(synthetic.device_blocks(N, K, seed=i), layout=lay) for i in range(ring)]
        for M in BATCHES:
            x = synthetic.device_activations(M, K, seed=M)
            launches = max(4, min(2 * ring, 4096 // M))
            kernels = {}
            if M <= 64:
                kernels["lut23"] = lambda i: tq1_matmul_words(weights[i % ring], x, layout=lay, config=MatmulConfig())
                kernels["direct"] = lambda i: tq1_gemm_words(weights[i % ring], x, layout=lay,
                                                             config=GemmConfig(form="direct"))
            kernels["wide"] = lambda i: tq1_gemm_words(weights[i % ring], x, layout=lay,
                                                       config=GemmConfig(form="wide"))
            kernels["tile"] = lambda i: tq1_gemm_words(weights[i % ring], x, layout=lay,
                                                       config=GemmConfig(form="tile"))
            times = {k: round(graph_us(fn, launches), 2) for k, fn in kernels.items()}
            rows.append({"shape": name, "K": K, "N": N, "M": M, "us": times})
            print(json.dumps(rows[-1]), flush=True)
            del x
        del weights
    Path(out).write_text(json.dumps({
        "device": torch.cuda.get_device_name(0),
        "method": "cold weight ring (>= 700 MB), launches replayed from one HIP graph, events around it",
        "rows": rows,
    }, indent=1) + "\n")


if __name__ == "__main__":
    main(sys.argv[1])
