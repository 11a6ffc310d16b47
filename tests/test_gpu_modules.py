"""Embedding gather and the module API (PackedLinear / PackedEmbedding /
matmul_words) on the GPU, against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, random_blocks, to_dev
from ternel_amd.format import FormatError
from ternel_amd import _lib
from ternel_amd.kernels import tq1_get_rows_words, tq1_get_rows_canonical
from ternel_amd.layout import pack_blocks
from ternel_amd.modules import PackedEmbedding, PackedLinear, matmul_words, replace_with_packed, select_kernel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(("rows", "columns"), ((1024, 5120), (48, 384), (300, 256)))
@pytest.mark.parametrize("dtype", (torch.float32, torch.float16))
def test_get_rows_is_bit_exact(rows: int, columns: int, dtype) -> None:
    blocks = random_blocks(rows, columns, seed=rows + 3)
    rng = np.random.default_rng(rows)
    ids = np.unique(np.concatenate([[0, rows - 1, rows // 2], rng.integers(0, rows, size=16)])).astype(np.int64)
    got = tq1_get_rows_words(pack(blocks), to_dev(ids), layout=layout(rows, columns), dtype=dtype)
    want = O.get_rows_reference(blocks, ids, rows=rows, columns=columns,
                                dtype=np.float32 if dtype == torch.float32 else np.float16)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_get_rows_bf16_rounds_the_exact_value_once() -> None:
    blocks = random_blocks(300, 256, seed=9)
    ids = np.arange(0, 300, 7, dtype=np.int64)
    got = tq1_get_rows_words(pack(blocks), to_dev(ids), layout=layout(300, 256), dtype=torch.bfloat16)
    want = O.get_rows_reference(blocks, ids, rows=300, columns=256, dtype=np.float32)
    np.testing.assert_array_equal(got.float().cpu().numpy(), torch.from_numpy(want).to(torch.bfloat16).float().numpy())


def test_get_rows_repeats_and_out_of_range_ids() -> None:
    blocks = random_blocks(512, 256, seed=44)
    ids = torch.tensor([7, 7, 511, 0, 7, 512, 100000, -1], dtype=torch.int64, device="cuda")
    got = tq1_get_rows_words(pack(blocks), ids, layout=layout(512, 256), dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(got[0], got[1])
    np.testing.assert_array_equal(got[0], got[4])
    assert not got[5:].any()
    assert got[2].any() and got[3].any()


@pytest.mark.parametrize(("rows", "columns"), ((1024, 5120), (300, 256), (64, 128)))
@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
def test_canonical_gather_is_bit_identical_to_the_packed_one(rows: int, columns: int, dtype) -> None:
    """Both table layouts give the same bits, including repeats, both ends of every block
    (runs 14 and 15 read the last word) and ids outside the table (zeros)."""
    blocks = random_blocks(rows, columns, seed=rows + columns)
    rng = np.random.default_rng(rows)
    ids = torch.tensor(np.concatenate([[0, rows - 1, 3, 3, rows, -5], rng.integers(0, rows, size=61)]),
                       dtype=torch.int64, device="cuda")
    lay = layout(rows, columns)
    canonical = torch.from_numpy(blocks).cuda()
    got = tq1_get_rows_canonical(canonical, ids, layout=lay, dtype=dtype)
    packed = tq1_get_rows_words(pack(blocks), ids, layout=lay, dtype=dtype)
    assert torch.equal(got.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       packed.view(torch.int16 if dtype != torch.float32 else torch.int32))
    assert not got[4:6].any()
    if dtype != torch.bfloat16:
        host_ids = ids[:4].cpu().numpy()
        want = O.get_rows_reference(blocks, host_ids, rows=rows, columns=columns,
                                    dtype=np.float32 if dtype == torch.float32 else np.float16)
        np.testing.assert_array_equal(got[:4].cpu().numpy(), want)


@pytest.mark.parametrize("entry", ("packed", "canonical"))
def test_gather_into_an_unaligned_output(entry: str) -> None:
    """An output that is not 16-byte aligned takes element stores, with the same values."""
    rows, columns = 300, 256
    blocks = random_blocks(rows, columns, seed=77)
    lay = layout(rows, columns)
    table = pack(blocks) if entry == "packed" else torch.from_numpy(blocks).cuda()
    ids = torch.tensor([5, 299, 0, 150], dtype=torch.int64, device="cuda")
    aligned = (tq1_get_rows_words if entry == "packed" else tq1_get_rows_canonical)(table, ids, layout=lay,
                                                                              dtype=torch.float16)
    buf = torch.zeros(ids.numel() * columns + 1, dtype=torch.float16, device="cuda")
    fn = _lib.lib().ternel_tq1_get_rows if entry == "packed" else _lib.lib().ternel_tq1_get_rows_canonical
    _lib.check(fn(table.data_ptr(), rows, columns, ids.data_ptr(), ids.numel(), buf[1:].data_ptr(),
                  _lib.DTYPE_F16, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert buf[0].item() == 0
    assert torch.equal(buf[1:].view(ids.numel(), columns).view(torch.int16), aligned.view(torch.int16))


def test_canonical_gather_rejects_a_wrong_table() -> None:
    lay = layout(256, 256)
    ids = torch.zeros(1, dtype=torch.int64, device="cuda")
    with pytest.raises(FormatError, match="canonical blocks"):
        tq1_get_rows_canonical(torch.zeros((256, 2, 27), dtype=torch.uint8, device="cuda"), ids, layout=lay,
                               dtype=torch.float32)


def test_get_rows_rejects_bad_indices() -> None:
    blocks = pack(random_blocks(256, 256, seed=1))
    with pytest.raises(FormatError, match="1-D"):
        tq1_get_rows_words(blocks, torch.zeros((2, 2), dtype=torch.int64, device="cuda"), layout=layout(256, 256),
                     dtype=torch.float32)
    with pytest.raises(FormatError, match="empty"):
        tq1_get_rows_words(blocks, torch.zeros((0,), dtype=torch.int64, device="cuda"), layout=layout(256, 256),
                     dtype=torch.float32)


def loaded_linear(rows: int, columns: int, seed: int) -> tuple[PackedLinear, np.ndarray]:
    blocks = random_blocks(rows, columns, seed=seed)
    lay = layout(rows, columns)
    module = PackedLinear(lay)
    codes, scales = pack_blocks(blocks, layout=lay)
    module.load_weights([("codes", codes), ("scales", scales)])
    return module, blocks


def test_packed_linear_loads_the_reference_tiled_arrays() -> None:
    module, blocks = loaded_linear(512, 640, seed=77)
    np.testing.assert_array_equal(module.blocks.cpu().numpy(), blocks)
    codes, scales = pack_blocks(blocks, layout=module.layout)
    np.testing.assert_array_equal(module.codes.cpu().numpy(), codes)
    np.testing.assert_array_equal(module.scales.cpu().numpy(), scales)


@pytest.mark.parametrize("batch", (1, 3, 16, 200))
def test_packed_linear_matches_the_oracle_in_every_dispatch_regime(batch: int) -> None:
    module, blocks = loaded_linear(512, 640, seed=batch)
    x = np.random.default_rng(batch).normal(0, 1, size=(batch, 640)).astype(np.float16)
    got = module(to_dev(x)).float().cpu().numpy()
    oracle = O.oracle_matmul(blocks, x.astype(np.float64), rows=512, columns=640)
    assert O.compare(got, oracle)["normalised_max_abs_error"] < 1e-3
    # 512 x 640 is under 16 MiB of packed weights: LUT23 up to 4 activation rows
    assert select_kernel(module.layout, batch, torch.float16) == ("lut23" if batch <= 4 else "gemm")


def test_packed_linear_keeps_leading_dimensions() -> None:
    module, _ = loaded_linear(256, 128, seed=77)
    x = torch.randn(2, 3, 128, device="cuda", dtype=torch.float16)
    out = module(x)
    assert tuple(out.shape) == (2, 3, 256)
    np.testing.assert_array_equal(out.reshape(-1, 256).cpu().numpy(), module(x.reshape(-1, 128)).cpu().numpy())


def test_packed_linear_rejects_a_wrong_width() -> None:
    module, _ = loaded_linear(256, 128, seed=1)
    with pytest.raises(FormatError, match="activation has 256 columns, weight expects 128"):
        module(torch.zeros(1, 256, device="cuda", dtype=torch.float16))


def test_loading_rejects_illegal_bytes() -> None:
    module, blocks = loaded_linear(256, 128, seed=2)
    bad = blocks.copy()
    bad[3, 0, 27] = 30
    with pytest.raises(FormatError, match="tail=1"):
        module.load_blocks(bad)


def test_packed_embedding_gathers_like_the_reference() -> None:
    rows, columns = 512, 256
    blocks = random_blocks(rows, columns, seed=909)
    lay = layout(rows, columns)
    module = PackedEmbedding(lay, dtype=torch.float32)
    module.load_blocks(blocks)
    tokens = torch.tensor([[0, 1, 255, 256], [rows - 1, 7, 128, 42]], dtype=torch.int32, device="cuda")
    out = module(tokens)
    assert tuple(out.shape) == (2, 4, columns)
    want = O.get_rows_reference(blocks, tokens.cpu().numpy().reshape(-1), rows=rows, columns=columns)
    np.testing.assert_array_equal(out.reshape(-1, columns).cpu().numpy(), want)


def test_tied_head_is_the_same_arithmetic_as_a_linear() -> None:
    rows, columns = 256, 128
    blocks = random_blocks(rows, columns, seed=31337)
    lay = layout(rows, columns)
    embedding = PackedEmbedding(lay, dtype=torch.float16)
    linear = PackedLinear(lay)
    embedding.load_blocks(blocks)
    linear.load_blocks(blocks)
    x = torch.randn(4, columns, device="cuda", dtype=torch.float16)
    np.testing.assert_array_equal(embedding.as_linear(x).cpu().numpy(), linear(x).cpu().numpy())


def test_packed_embedding_gathers_from_reloaded_weights() -> None:
    """The row-major copy the gathers read follows the packed words when they are reloaded."""
    rows, columns = 256, 256
    module = PackedEmbedding(layout(rows, columns), dtype=torch.float32)
    tokens = torch.tensor([0, 17, 255], device="cuda")
    for seed in (1, 2):
        blocks = random_blocks(rows, columns, seed=seed)
        module.load_blocks(blocks)
        want = O.get_rows_reference(blocks, tokens.cpu().numpy(), rows=rows, columns=columns)
        np.testing.assert_array_equal(module(tokens).cpu().numpy(), want)


def test_out_of_range_token_reads_zero() -> None:
    rows, columns = 256, 128
    module = PackedEmbedding(layout(rows, columns), dtype=torch.float32)
    module.load_blocks(random_blocks(rows, columns, seed=5))
    out = module(torch.tensor([rows, rows + 1000, 0], device="cuda")).cpu().numpy()
    assert not out[0].any() and not out[1].any() and out[2].any()


def test_replace_with_packed_swaps_every_linear_and_embedding() -> None:
    model = nn.Sequential(nn.Embedding(512, 256), nn.Linear(256, 384, bias=False), nn.Linear(384, 128, bias=False))
    replace_with_packed(model)
    assert isinstance(model[0], PackedEmbedding)
    assert isinstance(model[1], PackedLinear) and model[1].layout.rows == 384
    assert isinstance(model[2], PackedLinear) and model[2].layout.columns == 384
    assert not any(isinstance(m, nn.Linear) for m in model.modules())


def test_packed_matmul_function_matches_the_module() -> None:
    module, blocks = loaded_linear(256, 384, seed=12)
    x = torch.randn(3, 384, device="cuda", dtype=torch.float16)
    np.testing.assert_array_equal(matmul_words(module.packed, x, layout=module.layout).cpu().numpy(),
                                  module(x).cpu().numpy())
