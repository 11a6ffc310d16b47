"""BASELINE shapes at full size (configs 1, 3 and the config-4 embedding table).

The oracle cannot densify a whole 27B-class matrix in seconds, so full-size
launches are checked on seeded row/column samples against the fp64 oracle and
through size-independent properties: linearity in the activations, and
agreement of the LUT23 and MFMA paths on the same weights.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from ternel_amd import synthetic
from ternel_amd.kernels import GemmConfig, MatmulConfig, pack_weights, tq1_gemm_words, tq1_get_rows_words, tq1_matmul_words
from ternel_amd.layout import PackedTensorLayout

pytestmark = pytest.mark.gpu

SHAPES_C1 = ((5120, 17408), (17408, 5120), (5120, 8192))  # (K, N): gate/up, down, QKV


def sampled_oracle(blocks_host: np.ndarray, x: np.ndarray, rows: np.ndarray, columns: int) -> np.ndarray:
    sub = blocks_host[rows]
    return O.oracle_matmul(sub, x.astype(np.float64), rows=len(rows), columns=columns)


@pytest.mark.parametrize(("K", "N"), SHAPES_C1)
def test_decode_gemv_at_27b_shapes(K: int, N: int) -> None:
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 1)
    packed = pack_weights(blocks, layout=lay)
    x = synthetic.device_activations(1, K, seed=7)
    y = tq1_matmul_words(packed, x, layout=lay).float().cpu().numpy()
    rng = np.random.default_rng(K + N)
    rows = np.sort(rng.choice(N, size=512, replace=False))
    want = sampled_oracle(blocks.cpu().numpy(), x.cpu().numpy(), rows, K)
    got = y[:, rows]
    assert O.compare(got, want)["normalised_max_abs_error"] < 1e-3
    # Linearity: y(2x) == 2 y(x) exactly (scaling by two is exact in every step,
    # including the fp16 store, for outputs in the fp16 normal range).
    y2 = tq1_matmul_words(packed, x * 2, layout=lay).float().cpu().numpy()
    normal = np.abs(y) >= 2.0 ** -14
    np.testing.assert_array_equal(y2[normal], 2 * y[normal])


@pytest.mark.parametrize(("K", "N"), ((5120, 17408), (17408, 5120)))
@pytest.mark.parametrize("M", (512,))
def test_prefill_gemm_at_27b_shapes(K: int, N: int, M: int) -> None:
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 3)
    x = synthetic.device_activations(M, K, seed=9, sigma=0.5)
    y = tq1_gemm_words(pack_weights(blocks, layout=lay), x, layout=lay, config=GemmConfig()).float().cpu().numpy()
    rng = np.random.default_rng(K * 3 + N)
    rows = np.sort(rng.choice(N, size=256, replace=False))
    samples = np.sort(rng.choice(M, size=32, replace=False))
    want = sampled_oracle(blocks.cpu().numpy(), x.cpu().numpy()[samples], rows, K)
    got = y[np.ix_(samples, rows)]
    assert O.compare(got, want)["normalised_max_abs_error"] < 1e-3


@pytest.mark.parametrize("M", (2, 8, 16, 64))
def test_small_batch_paths_agree_at_the_gate_shape(M: int) -> None:
    K, N = 5120, 17408
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 2)
    x = synthetic.device_activations(M, K, seed=M)
    packed = pack_weights(blocks, layout=lay)
    lut = tq1_matmul_words(packed, x, layout=lay, config=MatmulConfig()).float().cpu().numpy()
    mfma = tq1_gemm_words(packed, x, layout=lay, config=GemmConfig()).float().cpu().numpy()
    rows = np.sort(np.random.default_rng(M).choice(N, size=256, replace=False))
    want = sampled_oracle(blocks.cpu().numpy(), x.cpu().numpy(), rows, K)
    assert O.compare(lut[:, rows], want)["normalised_max_abs_error"] < 1e-3
    assert O.compare(mfma[:, rows], want)["normalised_max_abs_error"] < 1e-3
    assert O.compare(mfma, lut)["normalised_max_abs_error"] < 2e-3


def test_embedding_gather_from_the_config4_table() -> None:
    rows, columns = 151936, 5120
    lay = PackedTensorLayout.for_tensor(rows, columns)
    table = synthetic.device_blocks(rows, columns, seed=synthetic.SEED_BASE + 4)
    ids = torch.tensor([0, 1, 75967, rows - 1, 151935, 42], dtype=torch.int64, device="cuda")
    got = tq1_get_rows_words(pack_weights(table, layout=lay), ids, layout=lay, dtype=torch.float16).cpu().numpy()
    sub = table[ids].cpu().numpy()
    want = O.get_rows_reference(sub, np.arange(len(ids)), rows=len(ids), columns=columns, dtype=np.float16)
    np.testing.assert_array_equal(got, want)
