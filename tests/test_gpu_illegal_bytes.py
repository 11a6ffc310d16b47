"""The compute kernels on bytes that were never validated.

The reference guards this case with its SAFE clamp build and a test that the
kernels stay in bounds (src/ternel_mlx/kernels.py:305,316,635-638;
tests/test_mlx_kernels.py:546-559). Here every index the kernels derive from a
byte is bounded for all 256 values by construction, which tests/byte_bounds.cpp
checks on the CPU; this test runs every form over a weight whose first 128 rows
hold illegal code bytes (243..255) in every slot and illegal tail bytes
(27..255), beside rows of legal bytes. Each call must succeed, every output
must be finite (an illegal digit selects a weight of the same group's scale
table, or zero), and the legal rows must still match the fp64 oracle -- the
illegal rows share tiles, groups and workgroups with them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, random_blocks, to_dev
from ternel_amd.kernels import GemmConfig, MatmulConfig, tq1_gemm_words, tq1_matmul_words

pytestmark = pytest.mark.gpu

NORTH_STAR_TOLERANCE = 1e-3
ROWS, COLUMNS, DIRTY = 256, 2048, 128


def dirty_blocks() -> np.ndarray:
    blocks = random_blocks(ROWS, COLUMNS, seed=243)
    rows = np.arange(DIRTY)[:, None, None]
    groups = np.arange(COLUMNS // 128)[None, :, None]
    slots = np.arange(25)[None, None, :]
    blocks[:DIRTY, :, 2:27] = (243 + (rows + 3 * groups + slots) % 13).astype(np.uint8)
    blocks[:DIRTY, :, 27] = (27 + (rows[:, :, 0] * 7 + groups[:, :, 0]) % 229).astype(np.uint8)
    return blocks


def run(kind: str, packed: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    lay = layout(ROWS, COLUMNS)
    if kind == "lut23":
        return tq1_matmul_words(packed, x, layout=lay, config=MatmulConfig(batch_tile=1, k_split=1))
    if kind == "lut23_split":
        return tq1_matmul_words(packed, x, layout=lay, config=MatmulConfig(batch_tile=2, k_split=4))
    return tq1_gemm_words(packed, x, layout=lay, config=GemmConfig(form=kind))


@pytest.mark.parametrize(("kind", "batch"), (("lut23", 1), ("lut23_split", 3), ("direct", 8), ("direct", 40),
                                             ("wide", 64), ("tile", 64)))
def test_illegal_bytes_stay_finite_and_leave_legal_rows_exact(kind: str, batch: int) -> None:
    blocks = dirty_blocks()
    assert O.count_invalid(blocks.reshape(-1, 28)) == (DIRTY * (COLUMNS // 128) * 25, DIRTY * (COLUMNS // 128))
    packed = pack(blocks)
    x_np = np.random.default_rng(batch).normal(0.0, 1.0, size=(batch, COLUMNS)).astype(np.float16)
    got = run(kind, packed, to_dev(x_np))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(got).all())
    clean = got[:, DIRTY:].float().cpu().numpy()
    want = O.oracle_matmul(blocks[DIRTY:], x_np.astype(np.float64), rows=ROWS - DIRTY, columns=COLUMNS)
    assert O.compare(clean, want)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE
