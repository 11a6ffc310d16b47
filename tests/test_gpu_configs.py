"""Every BASELINE.json config through the HIP path at its stated workload and
dtype, against the CPU oracle.

* configs[0] -- M=1, K = N = 4096, fp16 activations, fp16 output: all 4096
  rows against the fp64 dense oracle (src/ternel_mlx/reference.py:171-177) and
  the per-row fp32 decode-then-dot reference GEMV
  (src/bonsai_tq1/reference.py:14-65, the BASELINE CPU arm's arithmetic).
* configs[2] -- M in {2, 4, 8, 16, 32, 64} over gate/up 5120->17408, down
  17408->5120 and QKV 5120->8192 through the library dispatch
  (ternel_tq1_linear), sampled rows against the fp64 oracle.
* configs[3] -- M = 2048 on both prefill shapes, sampled rows x samples.
* configs[4] -- the O projection 8192->5120 at M=1, and the fused SwiGLU
  gate+up 5120->2x17408 at M=1, sampled units against SiLU(g)*u of the fp64
  projections.

Synthetic data as BASELINE.md states it: trits i.i.d. P(-1, 0, +1) = (0.3,
0.4, 0.3), scales fp16(|N(0, 0.02)| + 1e-4), activations fp16 N(0, 1)
(N(0, 0.5) for configs[3]). Tolerance: the north star's 1e-3 per-case
normalised error, written in each test; fused SwiGLU combines two values each
rounded once to fp16, so twice that plus one fp16 step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from ternel_amd import synthetic
from ternel_amd.kernels import GemmConfig, pack_weights, tq1_gemm_words, tq1_linear_words, tq1_matmul_words
from ternel_amd.layout import PackedTensorLayout, interleave_gate_up
from ternel_amd.modules import PackedSwiGLU

pytestmark = pytest.mark.gpu

NORTH_STAR_TOLERANCE = 1e-3
C1_SHAPES = {"gate_up": (5120, 17408), "down": (17408, 5120), "qkv": (5120, 8192)}  # name: (K, N)


def sampled(blocks: torch.Tensor, x: np.ndarray, rows: np.ndarray, columns: int) -> np.ndarray:
    return O.oracle_matmul(blocks[torch.from_numpy(rows).to(blocks.device)].cpu().numpy(), x.astype(np.float64),
                           rows=len(rows), columns=columns)


def test_config0_fp16_gemv_against_the_oracle_and_the_reference_gemv() -> None:
    K = N = 4096
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.host_blocks(N, K, seed=synthetic.SEED_BASE + 0)
    x = synthetic.host_activations(1, K, seed=synthetic.SEED_BASE + 0)  # fp16
    assert x.dtype == np.float16
    y = tq1_matmul_words(pack_weights(blocks, layout=lay), torch.from_numpy(x).cuda(), layout=lay)
    assert y.dtype == torch.float16
    got = y.float().cpu().numpy()
    assert O.compare(got, O.oracle_matmul(blocks, x.astype(np.float64), rows=N, columns=K))[
        "normalised_max_abs_error"] < NORTH_STAR_TOLERANCE
    reference = O.reference_gemv(blocks, x[0].astype(np.float32), rows=N, columns=K)[None, :]
    assert O.compare(got, reference)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE


@pytest.mark.parametrize("M", (2, 4, 8, 16, 32, 64))
@pytest.mark.parametrize("name", tuple(C1_SHAPES))
def test_config2_small_batches_through_the_library_dispatch(name: str, M: int) -> None:
    K, N = C1_SHAPES[name]
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 2)
    x = synthetic.device_activations(M, K, seed=synthetic.SEED_BASE + 2 + M)
    got = tq1_linear_words(pack_weights(blocks, layout=lay), x, layout=lay).float().cpu().numpy()
    rows = np.sort(np.random.default_rng(N + M).choice(N, size=192, replace=False))
    want = sampled(blocks, x.cpu().numpy(), rows, K)
    result = O.compare(got[:, rows], want)
    assert result["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE, result
    assert result["pattern_mismatches"] == 0


@pytest.mark.parametrize("name", ("gate_up", "down"))
def test_config3_prefill_at_2048_rows(name: str) -> None:
    K, N = C1_SHAPES[name]
    M = 2048
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 3)
    x = synthetic.device_activations(M, K, seed=synthetic.SEED_BASE + 3, sigma=0.5)
    y = tq1_gemm_words(pack_weights(blocks, layout=lay), x, layout=lay, config=GemmConfig()).float().cpu().numpy()
    rng = np.random.default_rng(K + 3 * N)
    rows = np.sort(rng.choice(N, size=192, replace=False))
    samples = np.sort(np.concatenate([rng.choice(M, size=24, replace=False), [0, M - 1]]))
    want = sampled(blocks, x.cpu().numpy()[samples], rows, K)
    assert O.compare(y[np.ix_(samples, rows)], want)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE


def test_config4_o_projection_at_m1() -> None:
    K, N = 8192, 5120
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 4)
    x = synthetic.device_activations(1, K, seed=synthetic.SEED_BASE + 4)
    got = tq1_linear_words(pack_weights(blocks, layout=lay), x, layout=lay).float().cpu().numpy()
    rows = np.sort(np.random.default_rng(11).choice(N, size=512, replace=False))
    assert O.compare(got[:, rows], sampled(blocks, x.cpu().numpy(), rows, K))[
        "normalised_max_abs_error"] < NORTH_STAR_TOLERANCE


def test_config4_fused_swiglu_at_the_mlp_width() -> None:
    hidden, K = 17408, 5120
    gate = synthetic.device_blocks(hidden, K, seed=synthetic.SEED_BASE + 41).cpu().numpy()
    up = synthetic.device_blocks(hidden, K, seed=synthetic.SEED_BASE + 42).cpu().numpy()
    mlp = PackedSwiGLU(hidden, K)
    mlp.load_blocks(gate, up)
    x = synthetic.host_activations(1, K, seed=synthetic.SEED_BASE + 43)
    z = mlp(torch.from_numpy(x).cuda()).float().cpu().numpy()
    units = np.sort(np.random.default_rng(5).choice(hidden, size=384, replace=False))
    xd = x.astype(np.float64)
    g = O.oracle_matmul(gate[units], xd, rows=len(units), columns=K)
    u = O.oracle_matmul(up[units], xd, rows=len(units), columns=K)
    want = g / (1.0 + np.exp(-g)) * u
    result = O.compare(z[:, units], want)
    assert result["normalised_max_abs_error"] < 2 * NORTH_STAR_TOLERANCE + 2.0 ** -11, result
    # the fused weight is the row interleave of the two projections
    assert interleave_gate_up(gate[:2], up[:2]).shape == (4, K // 128, 28)
