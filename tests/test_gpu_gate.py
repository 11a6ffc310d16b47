"""A replica of the reference's A4 kernel gate (src/ternel_mlx/kernel_gate.py),
run through the gfx950 kernels.

Per GATE_SHAPE (kernel_gate.py:74-80): a tensor from the reference's generator
(uniform trits, N(0, 0.05) fp16 scales; seed SEED + rows + columns), its
whole-tile prefix of at most 1024 rows (:84-91, :502-506) checked against the
CPU references -- the LUT23-order product, the fp64 dense oracle and the
per-row decode-then-dot product on a stride of cases -- over 128 random
activation vectors plus the ten edge cases (1e18, alternating 1e18, 1e-30,
mixed magnitudes 10^+-12, one-hots, ...; :391-430), the five non-finite cases
(:433-449) for propagation, and float16 / bfloat16 narrowings of the random
cases (:614-641). Tolerances are the gate's (:105-114): 1e-6 for a LUT23 arm
against the LUT23-order reference when unsplit, 1e-5 against any other
reference or when split, 2e-3 / 1e-2 after a float16 / bfloat16 narrowing.

Arms: the LUT23 kernel one vector per workgroup and four, unsplit and at the
gate's coarsest and finest K splits (:478-492), the automatic configuration,
the library dispatch; the MFMA forms (direct, wide, tile) on float16
activations -- the matrix cores take float16, so those arms are held to the
float16 narrowing bound against the fp64 oracle of the same float16 inputs.
Full-shape agreement (:661-720): every arm over the whole tensor against the
four-vector LUT23 arm.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from ternel_amd import synthetic
from ternel_amd.format import BLOCK_SIZE, encode_tq1_blocks
from ternel_amd.kernels import GemmConfig, MatmulConfig, pack_weights, tq1_gemm_words, tq1_linear_words, tq1_matmul_words
from ternel_amd.layout import PackedTensorLayout

pytestmark = pytest.mark.gpu

SEED = 20260810
GATE_SHAPES = (("linear_attn.in_proj_a", 48, 5120), ("self_attn.k_proj", 1024, 5120),
               ("linear_attn.out_proj", 5120, 6144), ("mlp.gate_proj", 17408, 5120), ("lm_head", 248320, 5120))
RANDOM_CASES = 128
REFERENCE_ROW_BUDGET = 1024
RESTORED_SAMPLES = 8
ORACLE_RELATIVE_TOLERANCE = 1e-5
SAME_ORDER_RELATIVE_TOLERANCE = 1e-6
NARROWED_RELATIVE_TOLERANCE = {torch.float16: 2e-3, torch.bfloat16: 1e-2}

SINGLE = MatmulConfig(threads=256, batch_tile=1, padded_lut=True, safe_clamp=False, k_split=1)
BATCHED = MatmulConfig(threads=256, batch_tile=4, padded_lut=False, safe_clamp=False, k_split=1)


def prefix_blocks(rows: int, columns: int) -> tuple[np.ndarray, int]:
    """The reference's generator (kernel_gate.py:374-388) for the CPU-checked
    prefix: whole 256-row tiles (the tile is the row count when 256 does not
    divide it), at most REFERENCE_ROW_BUDGET rows."""
    layout = PackedTensorLayout.for_tensor(rows, columns)
    prefix_rows = max(1, min(layout.tiles, REFERENCE_ROW_BUDGET // layout.tile)) * layout.tile
    gen = np.random.default_rng(SEED + rows + columns)
    groups = prefix_rows * (columns // BLOCK_SIZE)
    scale_bits = gen.normal(0.0, 0.05, size=groups).astype(np.float16).view(np.uint8).reshape(-1, 2)
    trits = gen.integers(0, 3, size=(groups, BLOCK_SIZE), dtype=np.uint8)
    return encode_tq1_blocks(scale_bits, trits).reshape(prefix_rows, columns // BLOCK_SIZE, 28), prefix_rows


def activation_cases(columns: int) -> tuple[np.ndarray, tuple[str, ...]]:
    """kernel_gate.py:391-430: 128 N(0,1) vectors, then the ten edge cases."""
    gen = np.random.default_rng(SEED + columns)
    random = gen.normal(0.0, 1.0, size=(RANDOM_CASES, columns)).astype(np.float32)
    labels = [f"random_{i}" for i in range(RANDOM_CASES)]
    large, small = np.float32(1e18), np.float32(1e-30)
    idx = np.arange(columns)
    edges = {
        "zeros": np.zeros(columns, np.float32),
        "ones": np.ones(columns, np.float32),
        "alternating_signs": np.where(idx % 2 == 0, 1.0, -1.0).astype(np.float32),
        "single_hot_first": np.eye(1, columns, 0, dtype=np.float32)[0],
        "single_hot_last": np.eye(1, columns, columns - 1, dtype=np.float32)[0],
        "single_hot_tail": np.eye(1, columns, 125, dtype=np.float32)[0],
        "large_positive": np.full(columns, large, np.float32),
        "large_alternating": np.where(idx % 2 == 0, large, -large).astype(np.float32),
        "small_normal": np.full(columns, small, np.float32),
        "mixed_magnitudes": (gen.normal(0.0, 1.0, size=columns)
                             * np.float32(10.0) ** gen.integers(-12, 12, size=columns)).astype(np.float32),
    }
    labels.extend(edges)
    return np.concatenate([random, np.stack(list(edges.values()))]), tuple(labels)


def non_finite_cases(columns: int) -> np.ndarray:
    """kernel_gate.py:433-449."""
    cases = np.zeros((5, columns), np.float32)
    cases[0, :] = np.nan
    cases[1, :] = np.inf
    cases[2, 0] = np.nan
    cases[3, 125] = np.nan
    cases[4, columns - 1] = -np.inf
    return cases


def split_gate_cases(groups: int) -> tuple[int, ...]:
    """kernel_gate.py:495-507: the coarsest and finest splits."""
    divisors = [k for k in range(2, groups + 1) if groups % k == 0]
    return tuple(sorted({min(divisors), max(divisors)}))


def lut_arms(groups: int) -> dict[str, MatmulConfig]:
    arms = {"lut23_single": SINGLE, "lut23_batched": BATCHED}
    for name, base in (("lut23_single", SINGLE), ("lut23_batched", BATCHED)):
        for split in split_gate_cases(groups):
            arms[f"{name}_k{split}"] = MatmulConfig(threads=256, batch_tile=base.batch_tile, padded_lut=False,
                                                    safe_clamp=False, k_split=split)
    arms["auto"] = MatmulConfig()
    return arms


def pair_tolerance(arm: str, reference: str) -> float:
    """kernel_gate.py:469-493: only an unsplit LUT23 arm against the LUT23 order."""
    if reference == "lut23" and arm in ("lut23_single", "lut23_batched"):
        return SAME_ORDER_RELATIVE_TOLERANCE
    return ORACLE_RELATIVE_TOLERANCE


@functools.lru_cache(maxsize=8)
def references(rows: int, columns: int):
    blocks, prefix_rows = prefix_blocks(rows, columns)
    x, labels = activation_cases(columns)
    stride = max(1, len(x) // RESTORED_SAMPLES)
    refs = {
        "lut23": O.lut23_matmul(blocks, x, rows=prefix_rows, columns=columns),
        "oracle": O.oracle_matmul(blocks, x, rows=prefix_rows, columns=columns),
        "restored": np.stack([O.reference_gemv(blocks, x[i], rows=prefix_rows, columns=columns)
                              for i in range(0, len(x), stride)]),
    }
    with np.errstate(invalid="ignore"):
        non_finite = O.lut23_matmul(blocks, non_finite_cases(columns), rows=prefix_rows, columns=columns)
    return blocks, prefix_rows, x, labels, stride, refs, non_finite


def run_lut(packed, x: np.ndarray, lay, config: MatmulConfig, dtype=torch.float32) -> np.ndarray:
    out = tq1_matmul_words(packed, torch.from_numpy(x).cuda().to(dtype), layout=lay, config=config)
    return out.float().cpu().numpy()


@pytest.mark.parametrize(("name", "rows", "columns"), GATE_SHAPES, ids=[s[0] for s in GATE_SHAPES])
def test_lut23_arms_against_the_cpu_references(name: str, rows: int, columns: int) -> None:
    blocks, prefix_rows, x, labels, stride, refs, _ = references(rows, columns)
    lay = PackedTensorLayout.for_tensor(prefix_rows, columns)
    packed = pack_weights(blocks, layout=lay)
    failures = []
    for arm, config in lut_arms(columns // BLOCK_SIZE).items():
        got = run_lut(packed, x, lay, config)
        for ref_name, ref in refs.items():
            sel = got[::stride] if ref_name == "restored" else got
            result = O.compare(sel, ref)
            tol = pair_tolerance(arm, ref_name)
            if result["normalised_max_abs_error"] > tol or result["pattern_mismatches"]:
                failures.append((arm, ref_name, result, labels[result["worst_case"] * (stride if ref_name ==
                                                                                          "restored" else 1)]))
    got = tq1_linear_words(packed, torch.from_numpy(x).cuda(), layout=lay).cpu().numpy()
    result = O.compare(got, refs["oracle"])
    if result["normalised_max_abs_error"] > ORACLE_RELATIVE_TOLERANCE or result["pattern_mismatches"]:
        failures.append(("linear", "oracle", result, labels[result["worst_case"]]))
    assert not failures, failures


@pytest.mark.parametrize(("name", "rows", "columns"), GATE_SHAPES, ids=[s[0] for s in GATE_SHAPES])
def test_non_finite_activations_propagate_as_the_reference(name: str, rows: int, columns: int) -> None:
    blocks, prefix_rows, _, _, _, _, non_finite = references(rows, columns)
    lay = PackedTensorLayout.for_tensor(prefix_rows, columns)
    packed = pack_weights(blocks, layout=lay)
    cases = non_finite_cases(columns)
    for config in (SINGLE, BATCHED):
        result = O.compare(run_lut(packed, cases, lay, config), non_finite)
        assert result["pattern_mismatches"] == 0, result
        assert result["normalised_max_abs_error"] <= SAME_ORDER_RELATIVE_TOLERANCE, result


@pytest.mark.parametrize(("name", "rows", "columns"), GATE_SHAPES, ids=[s[0] for s in GATE_SHAPES])
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_narrowed_activations_round_once(name: str, rows: int, columns: int, dtype) -> None:
    """The narrowed input is exact in fp32, so the LUT23-order reference over it
    leaves only the final store to differ (kernel_gate.py:614-641)."""
    blocks, prefix_rows, x, _, _, _, _ = references(rows, columns)
    lay = PackedTensorLayout.for_tensor(prefix_rows, columns)
    packed = pack_weights(blocks, layout=lay)
    narrow = torch.from_numpy(x[:RANDOM_CASES]).to(dtype)
    want = O.lut23_matmul(blocks, narrow.float().numpy(), rows=prefix_rows, columns=columns)
    got = tq1_matmul_words(packed, narrow.cuda(), layout=lay, config=BATCHED).float().cpu().numpy()
    assert O.compare(got, want)["normalised_max_abs_error"] <= NARROWED_RELATIVE_TOLERANCE[dtype]


@pytest.mark.parametrize(("name", "rows", "columns"), GATE_SHAPES, ids=[s[0] for s in GATE_SHAPES])
@pytest.mark.parametrize("form", ("direct", "wide", "tile"))
def test_mfma_arms_against_the_oracle_on_float16_activations(name: str, rows: int, columns: int, form: str) -> None:
    blocks, prefix_rows, x, _, _, _, _ = references(rows, columns)
    lay = PackedTensorLayout.for_tensor(prefix_rows, columns)
    packed = pack_weights(blocks, layout=lay)
    cases = 64 if form == "direct" else RANDOM_CASES
    narrow = x[:cases].astype(np.float16)
    got = tq1_gemm_words(packed, torch.from_numpy(narrow).cuda(), layout=lay,
                         config=GemmConfig(form=form)).float().cpu().numpy()
    want = O.oracle_matmul(blocks, narrow.astype(np.float64), rows=prefix_rows, columns=columns)
    result = O.compare(got, want)
    assert result["normalised_max_abs_error"] <= NARROWED_RELATIVE_TOLERANCE[torch.float16], result
    assert result["pattern_mismatches"] == 0


@pytest.mark.parametrize(("name", "rows", "columns"), GATE_SHAPES, ids=[s[0] for s in GATE_SHAPES])
def test_full_shape_agreement_between_arms(name: str, rows: int, columns: int) -> None:
    """Every arm over the whole tensor against the four-vector LUT23 arm
    (kernel_gate.py:661-720): the rows the CPU prefix never reaches."""
    lay = PackedTensorLayout.for_tensor(rows, columns)
    packed = pack_weights(synthetic.device_blocks(rows, columns, seed=SEED + rows), layout=lay)
    x, _ = activation_cases(columns)
    baseline = run_lut(packed, x, lay, BATCHED)
    failures = []
    for arm, config in lut_arms(columns // BLOCK_SIZE).items():
        if arm == "lut23_batched":
            continue
        got = run_lut(packed, x, lay, config)
        tol = SAME_ORDER_RELATIVE_TOLERANCE if arm == "lut23_single" else ORACLE_RELATIVE_TOLERANCE
        result = O.compare(got, baseline)
        if result["normalised_max_abs_error"] > tol or result["pattern_mismatches"]:
            failures.append((arm, result))
    narrow = x[:RANDOM_CASES].astype(np.float16)
    fp16_baseline = run_lut(packed, narrow.astype(np.float32), lay, BATCHED)
    for form in ("direct", "wide", "tile"):
        cases = 64 if form == "direct" else RANDOM_CASES
        got = tq1_gemm_words(packed, torch.from_numpy(narrow[:cases]).cuda(), layout=lay,
                             config=GemmConfig(form=form)).float().cpu().numpy()
        result = O.compare(got, fp16_baseline[:cases])
        if result["normalised_max_abs_error"] > NARROWED_RELATIVE_TOLERANCE[torch.float16] or \
                result["pattern_mismatches"]:
            failures.append((form, result))
    assert not failures, failures
