"""LUT23 kernel (decode GEMV and small batches) against the oracle.

Unsplit launches follow the reference kernel's summation order exactly, so they
are compared bit for bit with ``lut23_matmul``; every launch is also held to the
fp64 oracle (1e-5 case-normalised, the reference gate; the north star's 1e-3 is
looser), and split launches are pinned with exact +/-1 arithmetic.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, positional_all_slots, positional_tail, random_blocks, to_dev
from ternel_amd.format import FormatError
from ternel_amd.kernels import MatmulConfig, tq1_matmul_words

pytestmark = pytest.mark.gpu

ORACLE_TOLERANCE = 1e-5      # src/ternel_mlx/kernel_gate.py:105
NORTH_STAR_TOLERANCE = 1e-3  # BASELINE.json north star (fp32 accumulation)


def run(blocks: np.ndarray, x: np.ndarray, *, batch_tile: int = 1, k_split: int = 1,
        dtype=torch.float32) -> np.ndarray:
    rows, g, _ = blocks.shape
    lay = layout(rows, g * 128)
    out = tq1_matmul_words(pack(blocks), to_dev(x).to(dtype), layout=lay,
                     config=MatmulConfig(batch_tile=batch_tile, k_split=k_split))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_all_243_regular_bytes_at_every_slot_are_exact() -> None:
    blocks, x, want = positional_all_slots()
    np.testing.assert_array_equal(run(blocks, x), want)


def test_all_27_tail_bytes_are_exact() -> None:
    blocks, x, want = positional_tail()
    np.testing.assert_array_equal(run(blocks, x), want)


def test_every_fp16_scale_pattern_reaches_the_output() -> None:
    """tests/test_mlx_kernels.py:156-180: 65,536 rows, one +1 weight, x[0] = 1."""
    rows = 1 << 16
    blocks = np.zeros((rows, 1, 28), dtype=np.uint8)
    blocks[:, 0, 0:2] = np.arange(rows, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 0, 2:27] = 121
    blocks[:, 0, 2] = 122  # trit 0 = 2 -> weight +1
    blocks[:, 0, 27] = 13
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, 0] = 1.0
    got = run(blocks, x)[0]
    with np.errstate(invalid="ignore"):
        want = np.arange(rows, dtype=np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    np.testing.assert_array_equal(got[finite], want[finite])
    assert np.isnan(got[np.isnan(want)]).all()
    np.testing.assert_array_equal(got[np.isinf(want)], want[np.isinf(want)])


# 1536 and 2560 columns (12 and 20 groups) run as 4-group sub-chunks with the
# next one's loads issued early, including an odd last sub-chunk.
SHAPES = ((48, 5120), (256, 640), (512, 384), (1024, 5120), (300, 256), (256, 1536), (320, 2560))


@pytest.mark.parametrize(("rows", "columns"), SHAPES)
@pytest.mark.parametrize("batch", (1, 2, 3, 8))
@pytest.mark.parametrize("batch_tile", (1, 2, 4))
def test_unsplit_kernel_is_bit_exact_against_the_lut23_oracle(rows, columns, batch, batch_tile) -> None:
    blocks = random_blocks(rows, columns, seed=rows * 31 + columns)
    rng = np.random.default_rng(rows + columns + batch)
    x = rng.normal(0.0, 1.0, size=(batch, columns)).astype(np.float32)
    got = run(blocks, x, batch_tile=batch_tile, k_split=1)
    np.testing.assert_array_equal(got, O.lut23_matmul(blocks, x, rows=rows, columns=columns))
    oracle = O.oracle_matmul(blocks, x, rows=rows, columns=columns)
    assert O.compare(got, oracle)["normalised_max_abs_error"] < ORACLE_TOLERANCE


@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
def test_activation_dtypes_round_once_at_the_store(dtype) -> None:
    blocks = random_blocks(256, 384, seed=13)
    rng = np.random.default_rng(13)
    raw = torch.from_numpy(rng.normal(0.0, 1.0, size=(3, 384)).astype(np.float32)).to(dtype)
    x = raw.float().numpy()
    lay = layout(256, 384)
    out = tq1_matmul_words(pack(blocks), raw.to("cuda"), layout=lay, config=MatmulConfig(batch_tile=1, k_split=1))
    assert out.dtype == dtype
    want = O.lut23_matmul(blocks, x, rows=256, columns=384)
    # Only the final store is narrowed: the result is the fp32 answer rounded once.
    np.testing.assert_array_equal(out.cpu().numpy() if dtype == torch.float32 else out.float().cpu().numpy(),
                                  torch.from_numpy(want).to(dtype).float().numpy())


@pytest.mark.parametrize("fill", (0.0, 1.0, -1.0, 65504.0, -65504.0, 6.103515625e-05, 1e-8))
def test_extreme_and_degenerate_activations_match(fill: float) -> None:
    blocks = random_blocks(256, 384, seed=29)
    x = np.full((2, 384), fill, dtype=np.float32)
    np.testing.assert_array_equal(run(blocks, x), O.lut23_matmul(blocks, x, rows=256, columns=384))


@pytest.mark.parametrize("bad", (np.nan, np.inf, -np.inf))
@pytest.mark.parametrize("position", (0, 125, 383))
def test_non_finite_activations_reach_every_row(bad: float, position: int) -> None:
    blocks = random_blocks(256, 384, seed=31)
    x = np.zeros((1, 384), dtype=np.float32)
    x[0, position] = bad
    got = run(blocks, x)
    assert int(np.count_nonzero(np.isfinite(got))) == 0
    want = O.lut23_matmul(blocks, x, rows=256, columns=384)
    assert O.compare(got, want)["pattern_mismatches"] == 0


GROUP_COUNTS = (40, 48, 136)


@pytest.mark.parametrize("groups", GROUP_COUNTS)
def test_every_k_split_is_exact_on_integer_data(groups: int) -> None:
    """tests/test_mlx_kernels.py:619-666: unit scales, +/-1 activations -> exact integers."""
    rows, columns = 256, groups * 128
    rng = np.random.default_rng(groups)
    scales = np.full(rows * groups, 1.0, dtype=np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(rows * groups, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, groups, 28)
    x = rng.choice((-1.0, 1.0), size=(3, columns)).astype(np.float32)
    whole = run(blocks, x, k_split=1)
    assert np.array_equal(whole, np.rint(whole))
    np.testing.assert_array_equal(whole, O.oracle_matmul(blocks, x, rows=rows, columns=columns))
    for k in (k for k in range(2, groups + 1) if groups % k == 0):
        np.testing.assert_array_equal(run(blocks, x, k_split=k), whole, err_msg=f"k_split={k}")


@pytest.mark.parametrize("groups", GROUP_COUNTS)
@pytest.mark.parametrize("batch_tile", (1, 4))
def test_a_split_stays_inside_the_fp32_summation_bound(groups: int, batch_tile: int) -> None:
    """tests/test_mlx_kernels.py:669-716: |err| <= (128 + G) eps |W||x| elementwise."""
    rows, columns = 256, groups * 128
    blocks = random_blocks(rows, columns, seed=groups * 7 + batch_tile)
    rng = np.random.default_rng(groups + batch_tile)
    x = rng.normal(0.0, 1.0, size=(4, columns)).astype(np.float32)
    oracle = O.oracle_matmul(blocks, x, rows=rows, columns=columns)
    weights = O.dense_weights(blocks, rows=rows, columns=columns)
    bound = (128 + groups) * float(np.finfo(np.float32).eps) * (np.abs(x.astype(np.float64)) @ np.abs(weights).T)
    for k in (1,) + tuple(k for k in (2, 4, 5, 8, 17, 34) if groups % k == 0):
        got = run(blocks, x, batch_tile=batch_tile, k_split=k)
        assert (np.abs(got - oracle) <= bound).all(), f"k_split={k}"


@pytest.mark.parametrize("k_split", (2, 8, 40))
def test_a_split_result_is_bit_identical_between_runs(k_split: int) -> None:
    blocks = random_blocks(256, 5120, seed=k_split + 900)
    x = np.random.default_rng(k_split).normal(0.0, 1.0, size=(2, 5120)).astype(np.float32)
    first = run(blocks, x, k_split=k_split)
    for _ in range(3):
        np.testing.assert_array_equal(run(blocks, x, k_split=k_split), first)


def test_a_split_that_does_not_divide_the_groups_is_rejected() -> None:
    blocks = random_blocks(256, 5120, seed=311)
    with pytest.raises(FormatError, match="does not divide the tensor's 40 groups"):
        run(blocks, np.zeros((1, 5120), dtype=np.float32), k_split=3)


def test_activation_checks_match_the_reference_messages() -> None:
    blocks = pack(random_blocks(256, 384, seed=1))
    lay = layout(256, 384)
    with pytest.raises(FormatError, match="activations have 256 columns, expected 384"):
        tq1_matmul_words(blocks, torch.zeros((1, 256), device="cuda"), layout=lay)
    with pytest.raises(FormatError, match="2-D"):
        tq1_matmul_words(blocks, torch.zeros((384,), device="cuda"), layout=lay)
    with pytest.raises(FormatError, match="empty batch"):
        tq1_matmul_words(blocks, torch.zeros((0, 384), device="cuda"), layout=lay)
    with pytest.raises(FormatError, match="activations must be one of"):
        tq1_matmul_words(blocks, torch.zeros((1, 384), device="cuda", dtype=torch.float64), layout=lay)


@pytest.mark.parametrize("batch", (1, 2, 5, 16))
def test_auto_configuration_meets_the_north_star_tolerance(batch: int) -> None:
    rows, columns = 2048, 5120
    blocks = random_blocks(rows, columns, seed=batch)
    x = np.random.default_rng(batch).normal(0, 1, size=(batch, columns)).astype(np.float16)
    got = tq1_matmul_words(pack(blocks), to_dev(x), layout=layout(rows, columns)).float().cpu().numpy()
    oracle = O.oracle_matmul(blocks, x.astype(np.float32), rows=rows, columns=columns)
    result = O.compare(got, oracle)
    assert result["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE
    assert result["pattern_mismatches"] == 0


# One vector with the split left automatic (the M = 1 decode path): K chunks
# of four or eight groups reduced in chunk order. The shapes cover a single
# group (no split), ragged rows, and K from 2 to 136 groups.
# Ragged row counts (4000 = 62.5 64-row tiles, 26240 rows of 5 groups) and the
# QKV shape among them.
AUTO_SHAPES = ((128, 128), (64, 256), (300, 640), (8192, 1024), (2048, 5120), (1024, 17408), (4096, 2048),
               (4096, 4096), (4000, 5120), (26240, 640), (8192, 5120))


def run_auto(blocks: np.ndarray, x: np.ndarray, dtype=torch.float32) -> torch.Tensor:
    rows, g, _ = blocks.shape
    out = tq1_matmul_words(pack(blocks), to_dev(x).to(dtype), layout=layout(rows, g * 128), config=MatmulConfig())
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize(("rows", "columns"), AUTO_SHAPES)
def test_auto_split_gemv_stays_inside_the_fp32_summation_bound(rows: int, columns: int) -> None:
    """|err| <= (128 + G) eps |W||x| elementwise, the bound of any split."""
    groups = columns // 128
    blocks = random_blocks(rows, columns, seed=rows + columns)
    x = np.random.default_rng(rows * columns).normal(0.0, 1.0, size=(1, columns)).astype(np.float32)
    got = run_auto(blocks, x).cpu().numpy()
    oracle = O.oracle_matmul(blocks, x, rows=rows, columns=columns)
    weights = O.dense_weights(blocks, rows=rows, columns=columns)
    bound = (128 + groups) * float(np.finfo(np.float32).eps) * (np.abs(x.astype(np.float64)) @ np.abs(weights).T)
    assert (np.abs(got - oracle) <= bound).all()
    assert O.compare(got, oracle)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE


@pytest.mark.parametrize(("rows", "columns"), AUTO_SHAPES)
def test_auto_split_gemv_is_exact_on_integer_data(rows: int, columns: int) -> None:
    """Unit scales and +/-1 activations: every partial and sum is an exact integer."""
    groups = columns // 128
    rng = np.random.default_rng(rows + 7 * columns)
    scales = np.full(rows * groups, 1.0, dtype=np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(rows * groups, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, groups, 28)
    x = rng.choice((-1.0, 1.0), size=(1, columns)).astype(np.float32)
    np.testing.assert_array_equal(run_auto(blocks, x).cpu().numpy(),
                                  O.oracle_matmul(blocks, x, rows=rows, columns=columns))


def test_auto_split_gemv_of_one_group_is_bit_exact_against_the_lut23_oracle() -> None:
    """One group per row leaves nothing to split: the reference order."""
    blocks = random_blocks(200, 128, seed=5)
    x = np.random.default_rng(5).normal(0.0, 1.0, size=(1, 128)).astype(np.float32)
    np.testing.assert_array_equal(run_auto(blocks, x).cpu().numpy(),
                                  O.lut23_matmul(blocks, x, rows=200, columns=128))


@pytest.mark.parametrize(("rows", "columns"), ((2048, 17408), (4000, 5120)))
def test_auto_split_gemv_is_bit_identical_between_runs(rows: int, columns: int) -> None:
    blocks = random_blocks(rows, columns, seed=77)
    x = np.random.default_rng(77).normal(0.0, 1.0, size=(1, columns)).astype(np.float32)
    first = run_auto(blocks, x).cpu().numpy()
    for _ in range(3):
        np.testing.assert_array_equal(run_auto(blocks, x).cpu().numpy(), first)


@pytest.mark.parametrize("rows", (1024, 4000))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_auto_split_gemv_rounds_once_at_the_store(dtype, rows: int) -> None:
    blocks = random_blocks(rows, 5120, seed=17)
    raw = torch.from_numpy(np.random.default_rng(17).normal(0.0, 1.0, size=(1, 5120)).astype(np.float32)).to(dtype)
    narrow = run_auto(blocks, raw.numpy() if dtype == torch.float16 else raw.float().numpy(), dtype=dtype)
    assert narrow.dtype == dtype
    wide = run_auto(blocks, raw.float().numpy())
    np.testing.assert_array_equal(narrow.float().cpu().numpy(), wide.to(dtype).float().cpu().numpy())


@pytest.mark.parametrize("rows", (1024, 4000))
@pytest.mark.parametrize("bad", (np.nan, np.inf, -np.inf))
@pytest.mark.parametrize("position", (0, 2600, 5119))
def test_auto_split_gemv_carries_non_finite_activations_to_every_row(bad: float, position: int, rows: int) -> None:
    blocks = random_blocks(rows, 5120, seed=31)
    x = np.zeros((1, 5120), dtype=np.float32)
    x[0, position] = bad
    got = run_auto(blocks, x).cpu().numpy()
    want = O.oracle_matmul(blocks, x, rows=rows, columns=5120)
    assert int(np.count_nonzero(np.isfinite(got))) == 0
    assert O.compare(got, want)["pattern_mismatches"] == 0


@pytest.mark.parametrize(("rows", "columns"), ((5120, 17408), (5120, 8192)))
def test_a_vector_sums_the_same_in_any_batch_and_workgroup_shape(rows: int, columns: int) -> None:
    """At M=1 these splits run 128-row workgroups (down: 340 of 256 rows would
    leave most CUs one and some two), at M=2 256-row ones: each row's chunk
    and block order is the same, so the first vector's outputs are identical.
    (batch_tile=1 keeps M=1 on this kernel: left automatic, one vector over
    more than 40 groups takes the split strip GEMV.)"""
    blocks = random_blocks(rows, columns, seed=rows + columns)
    x = np.random.default_rng(columns).normal(0.0, 1.0, size=(2, columns)).astype(np.float32)
    one = tq1_matmul_words(pack(blocks), to_dev(x[:1]), layout=layout(rows, columns),
                           config=MatmulConfig(batch_tile=1)).cpu().numpy()
    two = run_auto(blocks, x).cpu().numpy()
    np.testing.assert_array_equal(two[:1], one)
    oracle = O.oracle_matmul(blocks, x[:1], rows=rows, columns=columns)
    assert O.compare(one, oracle)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE
