"""Both MFMA forms (LDS weight tiles; weights decoded into operand registers)
against the fp64 oracle.

Weights decode to fp16 (t - 1) * scale exactly and fp16 x fp16 products are
exact in fp32, so the only roundings are the fp32 accumulation and the final
fp16 store. Each element is therefore held to one fp16 rounding of the oracle
plus an fp32 accumulation bound, and every case to the north star's 1e-3
case-normalised error.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, random_blocks, to_dev
from ternel_amd.format import FormatError
from ternel_amd.kernels import GemmConfig, tq1_gemm_words

pytestmark = pytest.mark.gpu

NORTH_STAR_TOLERANCE = 1e-3
FP16_UNIT_ROUNDOFF = 2.0 ** -11


FORMS = ("tile", "direct", "wide")


def run(blocks: np.ndarray, x16: np.ndarray, *, k_split: int = 0, form: str = "auto") -> np.ndarray:
    rows, g, _ = blocks.shape
    out = tq1_gemm_words(pack(blocks), to_dev(x16), layout=layout(rows, g * 128),
                   config=GemmConfig(k_split=k_split, form=form))
    torch.cuda.synchronize()
    return out.float().cpu().numpy().astype(np.float64)


def assert_fp16_faithful(got: np.ndarray, blocks: np.ndarray, x16: np.ndarray) -> None:
    rows, g, _ = blocks.shape
    columns = g * 128
    x = x16.astype(np.float64)
    oracle = O.oracle_matmul(blocks, x, rows=rows, columns=columns)
    weights = O.dense_weights(blocks, rows=rows, columns=columns)
    terms = np.abs(x) @ np.abs(weights).T
    accumulation = columns * float(np.finfo(np.float32).eps) * terms
    # fp16 store: half an ulp of the (accumulated) value, incl. subnormal spacing.
    store = FP16_UNIT_ROUNDOFF * (np.abs(oracle) + accumulation) + 2.0 ** -25
    assert (np.abs(got - oracle) <= accumulation + store).all()
    result = O.compare(got, oracle)
    assert result["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE
    assert result["pattern_mismatches"] == 0


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("offset", (0, 64))
def test_mfma_lane_layout_probe(form: str, offset: int) -> None:
    """Identity activations pick out single weights: y[m][n] = W[n][offset + m].

    A transposed operand, a wrong accumulator lane map or (direct form) a K
    order of the activations that differs from the weights' moves values to
    other positions, which this catches element by element.
    """
    rows, columns = 256, 512
    blocks = random_blocks(rows, columns, seed=11)
    x = np.zeros((64, columns), dtype=np.float16)
    x[np.arange(64), offset + np.arange(64)] = 1.0
    x[np.arange(64), 128 + offset + np.arange(64)] = 1.0  # second group: same positions
    got = run(blocks, x, form=form)
    weights = O.dense_weights(blocks, rows=rows, columns=columns).astype(np.float16).astype(np.float64)
    want = (weights[:, offset:offset + 64] + weights[:, 128 + offset:128 + offset + 64]).T
    np.testing.assert_array_equal(got, want.astype(np.float16).astype(np.float64))


SHAPES = ((48, 5120), (256, 640), (512, 384), (1024, 5120), (300, 256))


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize(("rows", "columns"), SHAPES)
@pytest.mark.parametrize("batch", (1, 5, 32, 33, 64, 130, 256))
def test_gemm_matches_the_oracle(form: str, rows: int, columns: int, batch: int) -> None:
    if form == "direct" and batch > 64:
        pytest.skip("the direct form takes at most 64 activation rows")
    blocks = random_blocks(rows, columns, seed=rows * 31 + columns)
    x = np.random.default_rng(rows + columns + batch).normal(0.0, 1.0, size=(batch, columns)).astype(np.float16)
    assert_fp16_faithful(run(blocks, x, form=form), blocks, x)


@pytest.mark.parametrize("form", ("tile", "direct"))
@pytest.mark.parametrize("k_split", (1, 2, 5, 8, 40))
def test_gemm_split_k_matches_the_oracle(form: str, k_split: int) -> None:
    blocks = random_blocks(384, 5120, seed=k_split)
    x = np.random.default_rng(k_split).normal(0.0, 0.5, size=(37, 5120)).astype(np.float16)
    assert_fp16_faithful(run(blocks, x, k_split=k_split, form=form), blocks, x)


@pytest.mark.parametrize("form", FORMS)
def test_gemm_split_k_is_exact_on_integer_data(form: str) -> None:
    rows, groups = 256, 40
    rng = np.random.default_rng(3)
    scales = np.full(rows * groups, 1.0, dtype=np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(rows * groups, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, groups, 28)
    x = rng.choice((-1.0, 1.0), size=(20, groups * 128)).astype(np.float16)
    want = O.oracle_matmul(blocks, x.astype(np.float64), rows=rows, columns=groups * 128)
    # Integer results up to 5120 in magnitude are exact in fp16 only below 2048;
    # compare through fp16 rounding of the exact answer.
    want16 = want.astype(np.float16).astype(np.float64)
    for k in ((1,) if form == "wide" else (1, 2, 4, 5, 8, 10, 20, 40)):
        np.testing.assert_array_equal(run(blocks, x, k_split=k, form=form), want16, err_msg=f"k_split={k}")


@pytest.mark.parametrize("form", FORMS)
def test_gemm_is_deterministic(form: str) -> None:
    blocks = random_blocks(512, 5120, seed=5)
    x = np.random.default_rng(5).normal(0, 1, size=(64, 5120)).astype(np.float16)
    split = 0 if form == "wide" else 8
    first = run(blocks, x, k_split=split, form=form)
    for _ in range(2):
        np.testing.assert_array_equal(run(blocks, x, k_split=split, form=form), first)


@pytest.mark.parametrize("form", FORMS)
def test_gemm_propagates_non_finite_activations(form: str) -> None:
    columns = 512
    blocks = random_blocks(256, columns, seed=7)
    x = np.zeros((3, columns), dtype=np.float16)
    x[0, 0] = np.nan
    x[1, 125] = np.inf
    x[2, columns - 1] = -np.inf
    got = run(blocks, x, form=form)
    want = O.oracle_matmul(blocks, x.astype(np.float64), rows=256, columns=columns)
    assert O.compare(got, want)["pattern_mismatches"] == 0


def test_gemm_rejects_other_dtypes_and_bad_splits() -> None:
    blocks = pack(random_blocks(256, 384, seed=1))
    lay = layout(256, 384)
    with pytest.raises(FormatError, match="does not divide the tensor's 3 groups"):
        tq1_gemm_words(blocks, torch.zeros((4, 384), device="cuda", dtype=torch.float16), layout=lay,
                 config=GemmConfig(k_split=2))
    with pytest.raises(FormatError, match="activations have 256 columns, expected 384"):
        tq1_gemm_words(blocks, torch.zeros((4, 256), device="cuda", dtype=torch.float16), layout=lay)
    with pytest.raises(FormatError, match="at most 64 activation rows"):
        tq1_gemm_words(blocks, torch.zeros((65, 384), device="cuda", dtype=torch.float16), layout=lay,
                 config=GemmConfig(form="direct"))
    with pytest.raises(FormatError, match="stream-K"):
        tq1_gemm_words(blocks, torch.zeros((4, 384), device="cuda", dtype=torch.float16), layout=lay,
                 config=GemmConfig(form="wide", k_split=3))


@pytest.mark.parametrize(("rows", "columns", "batch"),
                         ((256, 5120, 5), (512, 17408, 300), (4096, 2048, 129), (4096, 17408, 800)))
def test_wide_stream_k_reduces_every_tile(rows: int, columns: int, batch: int) -> None:
    """Stream-K with many contributors per tile (one 256-row tile of 40 groups
    spread over 40 workgroups; ragged activation tiles), each reduced in order.
    The last case has enough tiles (16 x 4 of 136 groups) for 256-wide
    activation tiles; the others run 32- to 128-wide ones."""
    blocks = random_blocks(rows, columns, seed=rows + batch)
    x = np.random.default_rng(batch).normal(0.0, 0.5, size=(batch, columns)).astype(np.float16)
    got = run(blocks, x, form="wide")
    assert_fp16_faithful(got, blocks, x)
    np.testing.assert_array_equal(run(blocks, x, form="wide"), got)  # deterministic


@pytest.mark.parametrize("form", FORMS)
def test_gemm_non_finite_scales_follow_ieee(form: str) -> None:
    """A zero trit times an inf/NaN scale is NaN, as (t - 1) * scale computes it."""
    rows, columns = 128, 512
    rng = np.random.default_rng(9)
    scale_values = np.full(rows * 4, 0.5, dtype=np.float16)
    scale_values[3] = np.inf
    scale_values[64] = -np.inf
    scale_values[130] = np.nan
    trits = rng.integers(0, 3, size=(rows * 4, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scale_values.view(np.uint8).reshape(-1, 2), trits).reshape(rows, 4, 28)
    x = rng.normal(0, 1, size=(4, columns)).astype(np.float16)
    got = run(blocks, x, form=form)
    want = O.oracle_matmul(blocks, x.astype(np.float64), rows=rows, columns=columns)
    assert O.compare(got, want)["pattern_mismatches"] == 0
