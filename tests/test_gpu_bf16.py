"""bf16 activations on the matrix cores (the wide form after scale_rows_kernel).

Each activation row is scaled by a power of two into fp16's range (exact for
bf16 values: their 8-bit significand fits fp16's 11 bits) and the fp32 sums
are scaled back and rounded once to bf16. Pinned against the fp64 oracle with
the reference's bf16 tolerance (src/ternel_mlx/kernel_gate.py:113, 1e-2) on
sampled rows at full size; exactly on integer data; on rows whose magnitudes
span far more than fp16's range; on non-finite activations (the oracle's
NaN/inf pattern); through the library's dispatch and the fused SwiGLU; and
against the LUT23 kernel on the same bf16 inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import dev, layout, pack, random_blocks, to_dev
from ternel_amd import _lib, synthetic
from ternel_amd.kernels import (GemmConfig, MatmulConfig, pack_weights, tq1_gemm_words, tq1_linear_words,
                                tq1_matmul_words, tq1_swiglu_words)
from ternel_amd.format import FormatError
from ternel_amd.layout import PackedTensorLayout

pytestmark = pytest.mark.gpu

BF16_TOLERANCE = 1e-2  # src/ternel_mlx/kernel_gate.py:113


def bf16_host(x: torch.Tensor) -> np.ndarray:
    return x.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize(("K", "N", "M"), ((5120, 17408, 512), (17408, 5120, 512), (5120, 8192, 100),
                                           (5120, 17408, 2048), (640, 300, 65)))
def test_bf16_wide_gemm_matches_the_oracle_on_sampled_rows(K, N, M) -> None:
    print(f"bf16 wide: K={K} N={N} M={M}", flush=True)
    lay = PackedTensorLayout.for_tensor(N, K)
    blocks = synthetic.device_blocks(N, K, seed=synthetic.SEED_BASE + 7)
    x = synthetic.device_activations(M, K, seed=11, sigma=0.5).to(torch.bfloat16)
    y = tq1_gemm_words(pack_weights(blocks, layout=lay), x, layout=lay, config=GemmConfig())
    assert y.dtype == torch.bfloat16
    y = y.float().cpu().numpy()
    rng = np.random.default_rng(K + N + M)
    rows = np.sort(rng.choice(N, size=min(N, 128), replace=False))
    samples = np.sort(rng.choice(M, size=min(M, 16), replace=False))
    want = O.oracle_matmul(blocks.cpu().numpy()[rows], bf16_host(x)[samples], rows=len(rows), columns=K)
    assert O.compare(y[np.ix_(samples, rows)], want)["normalised_max_abs_error"] < BF16_TOLERANCE


def test_bf16_integer_products_are_exact() -> None:
    """Small-integer activations (exact in bf16) and weights with scale 1:
    every product and sum is an integer below 2^8, so the bf16 result is exact."""
    rows, columns, batch = 256, 1024, 96
    rng = np.random.default_rng(3)
    trits = rng.integers(0, 3, size=(rows * 8, 128), dtype=np.uint8)
    trits[:, 8:] = 1  # weight 0 beyond the first 8 per block: |sum| stays small
    scales = np.tile(np.array([0x00, 0x3C], dtype=np.uint8), (rows * 8, 1))  # fp16 1.0
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, 8, 28)
    x = rng.integers(-3, 4, size=(batch, columns)).astype(np.float32)
    got = tq1_gemm_words(pack(blocks), to_dev(x).to(torch.bfloat16), layout=layout(rows, columns),
                         config=GemmConfig(form="wide"))
    want = O.oracle_matmul(blocks, x.astype(np.float64), rows=rows, columns=columns)
    assert np.abs(want).max() < 256
    np.testing.assert_array_equal(got.float().cpu().numpy(), want.astype(np.float32))


def test_rows_beyond_fp16_range_are_scaled_not_clipped() -> None:
    """Rows of magnitude 2^100, 2^-100 and a row spanning 2^-20 .. 2^20: the
    per-row power-of-two scaling keeps every one exact in fp16."""
    rows, columns = 512, 2048
    blocks = random_blocks(rows, columns, seed=19)
    rng = np.random.default_rng(19)
    base = rng.normal(0.0, 1.0, size=(80, columns))
    x = base.copy()
    x[0] *= 2.0 ** 100
    x[1] *= 2.0 ** -100
    x[2] *= 2.0 ** rng.integers(-20, 21, size=columns)
    xb = to_dev(x.astype(np.float32)).to(torch.bfloat16)
    got = tq1_gemm_words(pack(blocks), xb, layout=layout(rows, columns), config=GemmConfig()).float().cpu().numpy()
    want = O.oracle_matmul(blocks, bf16_host(xb), rows=rows, columns=columns)
    for r in range(80):
        assert O.compare(got[r:r + 1], want[r:r + 1])["normalised_max_abs_error"] < BF16_TOLERANCE, r


def test_non_finite_activations_follow_the_oracle() -> None:
    rows, columns = 256, 1024
    blocks = random_blocks(rows, columns, seed=29)
    x = np.random.default_rng(29).normal(0.0, 1.0, size=(70, columns)).astype(np.float32)
    x[0, 5] = np.inf
    x[1, 700] = -np.inf
    x[2, 9] = np.nan
    x[3, 3] = 3e38  # finite in bf16, beyond fp16: scaled, not overflowed
    xb = to_dev(x).to(torch.bfloat16)
    got = tq1_gemm_words(pack(blocks), xb, layout=layout(rows, columns), config=GemmConfig()).float().cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        want = O.oracle_matmul(blocks, bf16_host(xb), rows=rows, columns=columns)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(np.isinf(got), np.isinf(want))
    finite = np.isfinite(want)
    assert O.compare(got[finite[:, 0]][:, :], want[finite[:, 0]])["normalised_max_abs_error"] < BF16_TOLERANCE
    assert np.isfinite(got[3]).all()


def test_bf16_runs_the_matrix_cores_through_the_library_dispatch() -> None:
    rows, columns, batch = 1024, 2560, 64
    handle = _lib.lib()
    assert handle.ternel_tq1_linear_kernel(batch, rows, columns, _lib.DTYPE_BF16) == 3  # the wide form
    blocks = random_blocks(rows, columns, seed=31)
    packed = pack(blocks)
    xb = to_dev(np.random.default_rng(31).normal(0.0, 1.0, size=(batch, columns)).astype(np.float32)).to(torch.bfloat16)
    got = tq1_linear_words(packed, xb, layout=layout(rows, columns)).float().cpu().numpy()
    lut = tq1_matmul_words(packed, xb, layout=layout(rows, columns), config=MatmulConfig()).float().cpu().numpy()
    want = O.oracle_matmul(blocks, bf16_host(xb), rows=rows, columns=columns)
    assert O.compare(got, want)["normalised_max_abs_error"] < BF16_TOLERANCE
    # both paths round an fp32 sum (in different orders) to bf16 once: one
    # bf16 step apart, or fp32 reassociation where a row's sum cancels
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(lut), 2.0 ** -126))) - 7)
    assert (np.abs(got - lut) <= step + 1e-5 * np.abs(want).max(axis=1, keepdims=True)).all()


def test_bf16_fused_swiglu_on_the_matrix_cores() -> None:
    rows, columns, batch = 2048, 1024, 80
    blocks = random_blocks(rows, columns, seed=37)
    packed = pack(blocks)
    xb = to_dev(np.random.default_rng(37).normal(0.0, 1.0, size=(batch, columns)).astype(np.float32)).to(torch.bfloat16)
    z = tq1_swiglu_words(packed, xb, layout=layout(rows, columns))
    linear = tq1_linear_words(packed, xb, layout=layout(rows, columns)).float()
    gate, up = linear[:, 0::2], linear[:, 1::2]
    want = (gate / (1.0 + torch.exp(-gate)) * up).to(torch.bfloat16)
    diff = (z.float() - want.float()).abs()
    tol = want.float().abs().clamp_min(2.0 ** -126) * 2.0 ** -7
    assert bool((diff <= tol).all())


def test_bf16_takes_no_other_mfma_form() -> None:
    rows, columns, batch = 256, 640, 8
    blocks = random_blocks(rows, columns, seed=41)
    xb = torch.zeros((batch, columns), dtype=torch.bfloat16, device=dev())
    with pytest.raises(FormatError, match="wide GEMM form"):
        tq1_gemm_words(pack(blocks), xb, layout=layout(rows, columns), config=GemmConfig(form="tile"))
    handle = _lib.lib()
    out = torch.empty((batch, rows), dtype=torch.bfloat16, device=dev())
    rc = handle.ternel_tq1_gemm(pack(blocks).data_ptr(), xb.data_ptr(), out.data_ptr(), batch, rows, columns,
                                _lib.DTYPE_BF16, 2, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL
    assert "bf16 activations run the wide form" in _lib.last_error()


@pytest.mark.parametrize("batch", (64, 300))  # two blocks (x in its own order), eight (permuted copy)
def test_unaligned_bf16_activations_give_the_same_result(batch) -> None:
    """The row-scaling pass reads 16-byte chunks when x is 16-byte aligned and
    single values otherwise: both give the same copy, so the same outputs."""
    rows, columns = 1024, 2560
    blocks = random_blocks(rows, columns, seed=43)
    packed = pack(blocks)
    x = to_dev(np.random.default_rng(43).normal(0.0, 1.0, size=(batch, columns)).astype(np.float32)).to(torch.bfloat16)
    storage = torch.zeros(batch * columns + 8, dtype=torch.bfloat16, device=dev())
    shifted = storage[1:1 + batch * columns].view(batch, columns)
    shifted.copy_(x)
    assert shifted.data_ptr() % 16 != 0 and x.data_ptr() % 16 == 0
    lay = layout(rows, columns)
    aligned = tq1_gemm_words(packed, x, layout=lay, config=GemmConfig(form="wide"))
    unaligned = tq1_gemm_words(packed, shifted, layout=lay, config=GemmConfig(form="wide"))
    assert torch.equal(aligned.view(torch.int16), unaligned.view(torch.int16))
    want = O.oracle_matmul(blocks, bf16_host(x), rows=rows, columns=columns)
    assert O.compare(aligned.float().cpu().numpy(), want)["normalised_max_abs_error"] < BF16_TOLERANCE
