"""The in-launch split-K fix-ups: the M = 1 decode GEMV (LUT23 kernel, K
chunks summed in chunk order by the last workgroup to arrive) at the 27B
shapes and tall or ragged ones, against the fp64 oracle and the fp32
summation bound; exact integers; bit identity between runs; the wide GEMM's
bounded stream-K wait driven to give up from the host; two streams at once,
each with its own workspace.

Pinned by: the fp64 dense product (oracle_matmul, src/ternel_mlx/reference.py:
171-177) with the per-case normalised tolerance of the north star; exact
integers on +/-1 data (every summation order agrees); bit identity between
runs (the reference's determinism contract, src/ternel_mlx/kernels.py:1232-1235).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import dev, layout, pack, random_blocks, to_dev
from ternel_amd import _lib
from ternel_amd.kernels import (GemmConfig, MatmulConfig, check_workspaces, tq1_gemm_words, tq1_matmul_words,
                                tq1_swiglu_words, workspace_errors)

pytestmark = pytest.mark.gpu

NORTH_STAR_TOLERANCE = 1e-3


def gemv(blocks: np.ndarray, x: np.ndarray, dtype=torch.float32) -> np.ndarray:
    rows, g, _ = blocks.shape
    out = tq1_matmul_words(pack(blocks), to_dev(x).to(dtype), layout=layout(rows, g * 128), config=MatmulConfig())
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


# (rows, columns): the three configs[1] matrices and their transposes, ragged
# last tiles, and a tall matrix (1024 row blocks x 5 chunks).
STREAM_SHAPES = ((17408, 5120), (5120, 17408), (8192, 5120), (5120, 8192), (4000, 2560), (1000, 640),
                 (65536, 2560))


@pytest.mark.parametrize(("rows", "columns"), STREAM_SHAPES)
def test_split_gemv_meets_the_fp32_bound_on_sampled_rows(rows: int, columns: int) -> None:
    groups = columns // 128
    blocks = random_blocks(rows, columns, seed=rows ^ columns)
    x = np.random.default_rng(rows + columns).normal(0.0, 1.0, size=(1, columns)).astype(np.float32)
    got = gemv(blocks, x)
    sample = np.unique(np.concatenate([np.arange(min(rows, 128)), np.arange(max(0, rows - 128), rows),
                                       np.random.default_rng(1).integers(0, rows, size=512)]))
    want = O.oracle_matmul(blocks[sample], x, rows=len(sample), columns=columns)
    weights = O.dense_weights(blocks[sample], rows=len(sample), columns=columns)
    bound = (128 + groups) * float(np.finfo(np.float32).eps) * (np.abs(x.astype(np.float64)) @ np.abs(weights).T)
    assert (np.abs(got[:, sample] - want) <= bound).all()
    assert O.compare(got[:, sample], want)["normalised_max_abs_error"] < NORTH_STAR_TOLERANCE


@pytest.mark.parametrize(("rows", "columns"), STREAM_SHAPES)
def test_split_gemv_is_exact_on_integer_data(rows: int, columns: int) -> None:
    groups = columns // 128
    rng = np.random.default_rng(rows + 3 * columns)
    scales = np.full(rows * groups, 1.0, dtype=np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(rows * groups, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, groups, 28)
    x = rng.choice((-1.0, 1.0), size=(1, columns)).astype(np.float32)
    # exact: |sum| <= 5120 * 17408-wide sums stay far inside fp32's integers
    want = (trits.reshape(rows, columns).astype(np.int64) - 1) @ x[0].astype(np.int64)
    np.testing.assert_array_equal(gemv(blocks, x)[0], want.astype(np.float32))


@pytest.mark.parametrize(("rows", "columns"), ((17408, 5120), (5120, 17408), (65536, 2560)))
def test_split_gemv_is_bit_identical_between_runs(rows: int, columns: int) -> None:
    blocks = random_blocks(rows, columns, seed=11)
    x = np.random.default_rng(11).normal(0.0, 1.0, size=(1, columns)).astype(np.float16)
    first = gemv(blocks, x, torch.float16)
    for _ in range(3):
        np.testing.assert_array_equal(gemv(blocks, x, torch.float16), first)
    assert not any(workspace_errors().values())


def test_fused_swiglu_gemv_at_the_27b_mlp_width() -> None:
    """gate + up 5120 -> 2 x 17408 as one interleaved weight, M = 1."""
    hidden, columns = 17408, 5120
    blocks = random_blocks(2 * hidden, columns, seed=3)
    x = np.random.default_rng(3).normal(0.0, 1.0, size=(1, columns)).astype(np.float16)
    lay = layout(2 * hidden, columns)
    z = tq1_swiglu_words(pack(blocks), to_dev(x), layout=lay).float().cpu().numpy()[0]
    y = gemv(blocks, x, torch.float16)[0]                       # the same rows, unfused
    g, u = torch.tensor(y[0::2]), torch.tensor(y[1::2])
    want = (torch.nn.functional.silu(g) * u).to(torch.float16).float().numpy()
    # SiLU's exp differs by a few ulp between the kernel and torch; one fp16 rounding apart at most
    np.testing.assert_allclose(z, want, rtol=2e-3, atol=1e-3 * float(np.abs(want).max()))


def test_split_gemv_on_two_streams_at_once() -> None:
    """Each stream has its own workspace: interleaved launches on two streams
    give each stream's result exactly (down 17408 -> 5120, a 17-way split)."""
    rows, columns = 5120, 17408
    blocks = [random_blocks(rows, columns, seed=s) for s in (21, 22)]
    xs = [np.random.default_rng(s).normal(0, 1, size=(1, columns)).astype(np.float16) for s in (21, 22)]
    packed = [pack(b) for b in blocks]
    xt = [to_dev(x) for x in xs]
    lay = layout(rows, columns)
    want = [tq1_matmul_words(p, x, layout=lay).cpu() for p, x in zip(packed, xt)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[], []]
    for _ in range(20):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i].append(tq1_matmul_words(packed[i], xt[i], layout=lay))
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert torch.equal(o.cpu(), want[i])
    check_workspaces()


def _wide_case():
    rows, columns, batch = 17408, 5120, 512
    blocks = random_blocks(rows, columns, seed=43)
    x = np.random.default_rng(43).normal(0, 0.5, size=(batch, columns)).astype(np.float16)
    packed, xt, lay = pack(blocks), to_dev(x), layout(rows, columns)
    config = GemmConfig(form="wide")
    want = tq1_gemm_words(packed, xt, layout=lay, config=config)  # also sizes the workspace eagerly
    torch.cuda.synchronize()
    return packed, xt, lay, config, want.cpu()


def _nan_tiles_and_exact_elsewhere(got: torch.Tensor, want: torch.Tensor) -> None:
    """The tiles whose reduction gave up (or was refused) are NaN, whole
    32-row x 256-column tiles of the wide form; every other value is the
    exact result -- nothing finite and wrong."""
    nan = torch.isnan(got.float())
    assert nan.any()
    assert torch.equal(got[~nan], want[~nan])
    m, n = got.shape
    tiles = nan[: m // 32 * 32, : n // 256 * 256].reshape(m // 32, 32, n // 256, 256)
    assert bool((tiles.all(dim=3).all(dim=1) == tiles.any(dim=3).any(dim=1)).all())


def test_a_wide_reduction_that_gives_up_writes_nan_tiles_and_the_next_call_raises() -> None:
    packed, xt, lay, config, want = _wide_case()
    handle = _lib.lib()
    # A negative limit makes every bounded wait give up at once (host-driven:
    # every kernel still exits normally; the other contributors publish late).
    old = handle.ternel_tq1_set_spin_limit(-1)
    try:
        got = tq1_gemm_words(packed, xt, layout=lay, config=config)
        torch.cuda.synchronize()
    finally:
        handle.ternel_tq1_set_spin_limit(old)
    _nan_tiles_and_exact_elsewhere(got.cpu(), want)
    assert any(w & 2 for w in workspace_errors().values())
    # The next call on that workspace raises before launching, and zeroes it.
    with pytest.raises(_lib.NativeError, match="bounded wait"):
        tq1_gemm_words(packed, xt, layout=lay, config=config)
    assert not any(workspace_errors().values())
    assert torch.equal(tq1_gemm_words(packed, xt, layout=lay, config=config).cpu(), want)


def test_a_workspace_whose_error_word_is_set_is_refused_by_the_kernel() -> None:
    """Called through the C ABI (no host-side check), a launch on a workspace
    left with its error word set -- stale counters -- writes the tiles that
    need them as NaN and leaves every other tile exact, launch after launch,
    until the workspace is zeroed."""
    packed, xt, lay, config, want = _wide_case()
    handle = _lib.lib()
    rows, columns = lay.rows, lay.columns
    batch = xt.shape[0]
    need = handle.ternel_tq1_gemm_workspace_bytes(batch, rows, columns, 3, 0)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev())
    ws[64 * 1024 - 4:64 * 1024].view(torch.int32).fill_(2)
    out = torch.empty((batch, rows), dtype=torch.float16, device=dev())

    def launch() -> None:
        _lib.check(handle.ternel_tq1_gemm(packed.data_ptr(), xt.data_ptr(), out.data_ptr(), batch, rows, columns,
                                          _lib.DTYPE_F16, 3, 0, ws.data_ptr(), ws.numel(),
                                          torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()

    launch()
    _nan_tiles_and_exact_elsewhere(out.cpu(), want)
    assert int(ws[64 * 1024 - 4:64 * 1024].view(torch.int32).item()) == 2  # still refused until zeroed
    launch()
    _nan_tiles_and_exact_elsewhere(out.cpu(), want)
    ws.zero_()
    launch()
    assert torch.equal(out.cpu(), want)
    assert ws[: 64 * 1024].eq(0).all()  # counters back at zero (the partial slots keep data)


def test_workspace_error_entry_refuses_a_workspace_without_an_error_word() -> None:
    handle = _lib.lib()
    word = ctypes.c_int(0)
    buf = torch.zeros(1024, dtype=torch.uint8, device=dev())
    assert handle.ternel_tq1_workspace_error(buf.data_ptr(), 1024, ctypes.byref(word), None) == _lib.TERNEL_TQ1_EINVAL
