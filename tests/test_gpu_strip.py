"""The strip GEMV (one activation vector, strips of at most 96 rows per CU, at
most 40 groups per row) against the oracle.

The automatic configuration of ``tq1_matmul_words`` runs it for these shapes;
each test first checks, through the workspace query (the strip GEMV needs
none, the LUT23 kernel a split-K workspace), that the shape does take it.
Covered: staged fp16/bf16 activations, fp32 and unaligned fp16 activations
(read from global memory), strips of unequal and odd row counts, one group per
row, the 62-row edge, the fused SwiGLU form, exact integer arithmetic on every
code byte and tail byte, and run-to-run bit identity.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, random_blocks, to_dev
from tests.test_gpu_swiglu import spacing
from ternel_amd import _lib
from ternel_amd.kernels import MatmulConfig, tq1_matmul_words, tq1_swiglu_words

pytestmark = pytest.mark.gpu

ORACLE_TOLERANCE = 1e-5      # src/ternel_mlx/kernel_gate.py:105 (fp32 output)
NORTH_STAR_TOLERANCE = 1e-3  # BASELINE.json north star (fp16 output)
BF16_TOLERANCE = 1e-2        # src/ternel_mlx/kernel_gate.py:113 (bf16 output: 8-bit significand)
TOLERANCE = {torch.float32: ORACLE_TOLERANCE, torch.float16: NORTH_STAR_TOLERANCE, torch.bfloat16: BF16_TOLERANCE}


def takes_strip(rows: int, columns: int) -> bool:
    return _lib.lib().ternel_tq1_matmul_workspace_bytes(1, rows, columns, 0, 0) == 0


def run(blocks: np.ndarray, x: torch.Tensor) -> torch.Tensor:
    rows, g, _ = blocks.shape
    assert takes_strip(rows, g * 128), f"{rows}x{g * 128} does not take the strip GEMV on this device"
    out = tq1_matmul_words(pack(blocks), x, layout=layout(rows, g * 128), config=MatmulConfig())
    torch.cuda.synchronize()
    return out


# (rows, columns): QKV (20 items of 64 blocks per strip: waves 0-3 sum two,
# the rest one); gate/up (68-row strips: two waves add the row sums); 4096^2;
# one group; strips of 8 and 10 rows (2050 rows over 256 CUs) and an odd last
# strip; 62, 64 (one summing wave's edge) and 66 rows; the 96-row edge (24576
# rows); 12 groups; 16 items per strip (one per wave).
SHAPES = ((8192, 5120), (17408, 5120), (4096, 4096), (2048, 128), (2050, 640), (3001, 1024), (15872, 5120),
          (16384, 2560), (16896, 3072), (24576, 5120), (6144, 1536), (8192, 4096))


@pytest.mark.parametrize(("rows", "columns"), SHAPES)
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_strip_gemv_matches_the_oracle(rows, columns, dtype) -> None:
    print(f"strip: rows={rows} columns={columns} {dtype}", flush=True)
    blocks = random_blocks(rows, columns, seed=rows * 7 + columns)
    x = np.random.default_rng(rows + columns).normal(0.0, 1.0, size=(1, columns)).astype(np.float32)
    xd = to_dev(x).to(dtype)
    got = run(blocks, xd).float().cpu().numpy()
    oracle = O.oracle_matmul(blocks, xd.float().cpu().numpy().astype(np.float64), rows=rows, columns=columns)
    assert O.compare(got, oracle)["normalised_max_abs_error"] < TOLERANCE[dtype]


def test_unaligned_fp16_activations_are_read_from_global_memory() -> None:
    rows, columns = 8192, 5120
    blocks = random_blocks(rows, columns, seed=17)
    x = np.random.default_rng(17).normal(0.0, 1.0, size=(1, columns)).astype(np.float16)
    storage = torch.zeros(columns + 8, dtype=torch.float16, device="cuda")
    view = storage[3:3 + columns].view(1, columns)
    view.copy_(to_dev(x))
    assert view.data_ptr() % 16 != 0
    got = run(blocks, view)
    aligned = run(blocks, to_dev(x))
    # the same tables and sums either way
    assert torch.equal(got.view(torch.int16), aligned.view(torch.int16))
    oracle = O.oracle_matmul(blocks, x.astype(np.float64), rows=rows, columns=columns)
    assert O.compare(got.float().cpu().numpy(), oracle)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE


def test_every_code_byte_and_tail_byte_is_exact() -> None:
    """Row p (of 2187 = 9 x 243) holds byte p % 243 in every one of its 25
    slots of group s = slot, and tail byte p % 27; x carries 1, 3, 9, 27, 81 in
    slot s of group s (and 1, 3, 9 in the tail of group 0), so row p is
    25 (p % 243 - 121) + (p % 27 - 13), exact in fp32."""
    rows, groups = 2187, 25
    blocks = np.zeros((rows, groups, 28), dtype=np.uint8)
    blocks[:, :, 0], blocks[:, :, 1] = 0x00, 0x3C  # scale 1.0
    p = np.arange(rows)
    blocks[:, :, 2:27] = (p % 243)[:, None, None]
    blocks[:, :, 27] = (p % 27)[:, None]
    x = np.zeros((1, groups * 128), dtype=np.float32)
    for s in range(groups):
        x[0, s * 128 + 5 * s: s * 128 + 5 * s + 5] = (1, 3, 9, 27, 81)
    x[0, 125:128] = (1, 3, 9)
    got = run(blocks, to_dev(x)).cpu().numpy()[0]
    want = 25.0 * (p % 243 - 121) + (p % 27 - 13)
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_results_are_bit_identical_from_run_to_run() -> None:
    rows, columns = 8192, 5120
    blocks = random_blocks(rows, columns, seed=5)
    packed = pack(blocks)
    x = to_dev(np.random.default_rng(5).normal(0.0, 1.0, size=(1, columns)).astype(np.float16))
    assert takes_strip(rows, columns)
    outs = [tq1_matmul_words(packed, x, layout=layout(rows, columns), config=MatmulConfig()) for _ in range(4)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("rows", (12288, 20480))  # 48- and 80-row strips (one and two summing waves)
def test_fused_swiglu_form(dtype, rows) -> None:
    """Rows alternate gate, up; the kernel writes SiLU(gate) * up from the two
    outputs rounded to the activation type."""
    columns = 5120
    assert takes_strip(rows, columns)
    blocks = random_blocks(rows, columns, seed=23)
    x = to_dev(np.random.default_rng(23).normal(0.0, 1.0, size=(1, columns)).astype(np.float32)).to(dtype)
    z = tq1_swiglu_words(pack(blocks), x, layout=layout(rows, columns))
    linear = tq1_matmul_words(pack(blocks), x, layout=layout(rows, columns), config=MatmulConfig())
    torch.cuda.synchronize()
    gate, up = linear[:, 0::2].float(), linear[:, 1::2].float()
    want = (gate / (1.0 + torch.exp(-gate)) * up).to(dtype).float()
    got = z.float()
    # one step of the activation type apart at most (the kernel's expf vs torch.exp)
    assert bool(((got - want).abs() <= spacing(want, dtype)).all())
    oracle = O.oracle_matmul(blocks, x.float().cpu().numpy().astype(np.float64), rows=rows, columns=columns)
    g64, u64 = oracle[:, 0::2], oracle[:, 1::2]
    ref = g64 / (1.0 + np.exp(-g64)) * u64
    assert O.compare(got.cpu().numpy(), ref)["normalised_max_abs_error"] < 4 * TOLERANCE[dtype]


# --- rows of more than 40 groups: the strip GEMV in Z = ceil(G / 40) <= 4 K
# chunks, one workgroup per (strip, chunk), S = CUs / Z strips; a row's chunk
# partials meet in a fixed tree of exchange slots in the workspace's counter
# region, (c0 + c1), ((c0 + c1) + c2) or ((c0 + c1) + (c2 + c3)).

COUNTERS = 64 * 1024  # the workspace's counter region


def takes_split_strip(rows: int, columns: int, chunks: int) -> bool:
    # the (tile, group) kernel's split needs partials past the counter region
    assert chunks == -(-columns // 128 // 40)
    return _lib.lib().ternel_tq1_matmul_workspace_bytes(1, rows, columns, 0, 0) == COUNTERS


def run_split(blocks: np.ndarray, x: torch.Tensor, chunks: int) -> torch.Tensor:
    rows, g, _ = blocks.shape
    assert takes_split_strip(rows, g * 128, chunks), f"{rows}x{g * 128} does not take the split strip GEMV"
    out = tq1_matmul_words(pack(blocks), x, layout=layout(rows, g * 128), config=MatmulConfig())
    torch.cuda.synchronize()
    return out


# (rows, columns, chunks): O 8192 -> 5120 (2 x 32 groups, 40-row strips);
# down 17408 -> 5120 (4 x 34, 80 rows); out_proj 6144 -> 5120 (2 x 24); 41
# groups (chunks of 21 and 20) over an odd row count; 80 groups over 64-row
# strips (three items per wave); 96 groups (3 x 32, 85 strips); 112 groups
# (38, 38, 36) over an odd row count; 160 groups (4 x 40) over 16-row strips.
SPLIT_SHAPES = ((5120, 8192, 2), (5120, 17408, 4), (5120, 6144, 2), (3001, 5248, 2), (8192, 10240, 2),
                (4096, 12288, 3), (3001, 14336, 3), (2050, 20480, 4))


@pytest.mark.parametrize(("rows", "columns", "chunks"), SPLIT_SHAPES)
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_split_strip_gemv_matches_the_oracle(rows, columns, chunks, dtype) -> None:
    print(f"split strip: rows={rows} columns={columns} chunks={chunks} {dtype}", flush=True)
    blocks = random_blocks(rows, columns, seed=rows * 5 + columns)
    x = np.random.default_rng(rows + 3 * columns).normal(0.0, 1.0, size=(1, columns)).astype(np.float32)
    xd = to_dev(x).to(dtype)
    got = run_split(blocks, xd, chunks).float().cpu().numpy()
    oracle = O.oracle_matmul(blocks, xd.float().cpu().numpy().astype(np.float64), rows=rows, columns=columns)
    assert O.compare(got, oracle)["normalised_max_abs_error"] < TOLERANCE[dtype]


def test_split_strip_gemv_is_exact_on_integer_data() -> None:
    """Unit scales and +/-1 activations: every block sum, chunk partial and
    total is an exact integer, whatever the order."""
    rows, columns = 5120, 17408
    groups = columns // 128
    rng = np.random.default_rng(41)
    scales = np.full(rows * groups, 1.0, dtype=np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(rows * groups, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, groups, 28)
    x = rng.choice((-1.0, 1.0), size=(1, columns)).astype(np.float32)
    got = run_split(blocks, to_dev(x), 4).cpu().numpy()
    np.testing.assert_array_equal(got, O.oracle_matmul(blocks, x, rows=rows, columns=columns))


def test_split_strip_gemv_rearms_its_counters_and_repeats_bit_for_bit() -> None:
    """Back-to-back calls of shapes with different chunk counts and strip
    counts on the library's workspace: each call finds its exchange slots
    empty and leaves them so, and every repeat is bit-identical."""
    a = random_blocks(5120, 17408, seed=3)
    b = random_blocks(5120, 8192, seed=4)
    c = random_blocks(4096, 12288, seed=5)
    xa = to_dev(np.random.default_rng(3).normal(0.0, 1.0, size=(1, 17408)).astype(np.float16))
    xb = to_dev(np.random.default_rng(4).normal(0.0, 1.0, size=(1, 8192)).astype(np.float16))
    xc = to_dev(np.random.default_rng(5).normal(0.0, 1.0, size=(1, 12288)).astype(np.float16))
    first_a = run_split(a, xa, 4).view(torch.int16).clone()
    first_b = run_split(b, xb, 2).view(torch.int16).clone()
    first_c = run_split(c, xc, 3).view(torch.int16).clone()
    for _ in range(3):
        assert torch.equal(run_split(a, xa, 4).view(torch.int16), first_a)
        assert torch.equal(run_split(b, xb, 2).view(torch.int16), first_b)
        assert torch.equal(run_split(c, xc, 3).view(torch.int16), first_c)


def test_split_strip_gemv_unaligned_activations_give_the_same_result() -> None:
    rows, columns = 5120, 8192
    blocks = random_blocks(rows, columns, seed=23)
    x = np.random.default_rng(23).normal(0.0, 1.0, size=(1, columns)).astype(np.float16)
    storage = torch.zeros(columns + 8, dtype=torch.float16, device="cuda")
    view = storage[5:5 + columns].view(1, columns)
    view.copy_(to_dev(x))
    assert view.data_ptr() % 16 != 0
    assert torch.equal(run_split(blocks, view, 2).view(torch.int16), run_split(blocks, to_dev(x), 2).view(torch.int16))
