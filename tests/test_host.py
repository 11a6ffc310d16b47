"""Host logic (CPU only): layout API, host encoder, synthetic generators, and the
C-ABI library loading with every symbol include/ternel_tq1.h declares.

Nothing here launches a kernel.
"""

from __future__ import annotations

import ctypes
import json
import re

import numpy as np
import pytest

from oracle import tq1_oracle as O
from tests.conftest import GOLDEN, ROOT
from ternel_amd import _lib
from ternel_amd.format import BLOCK_BYTES, BLOCK_SIZE, CODE_SLOTS, FormatError, encode_tq1_blocks
from ternel_amd.layout import (
    LAYOUT_NAME,
    MODEL_LINEAR_SHAPES,
    PREFERRED_TILE,
    SCALE_BYTES,
    PackedTensorLayout,
    pack_blocks,
    select_tile,
    unpack_blocks,
)
from ternel_amd import synthetic

KAT = json.loads((GOLDEN / "known_answers.json").read_text())

# tests/test_mlx_format.py:13-30
MODEL_TENSOR_SHAPES = (
    ("embed_tokens", 248320, 5120), ("lm_head", 248320, 5120),
    ("linear_attn.in_proj_a", 48, 5120), ("linear_attn.in_proj_b", 48, 5120),
    ("linear_attn.in_proj_qkv", 10240, 5120), ("linear_attn.in_proj_z", 6144, 5120),
    ("linear_attn.out_proj", 5120, 6144), ("self_attn.q_proj", 12288, 5120),
    ("self_attn.k_proj", 1024, 5120), ("self_attn.v_proj", 1024, 5120),
    ("self_attn.o_proj", 5120, 12288), ("mlp.gate_proj", 17408, 5120),
    ("mlp.up_proj", 17408, 5120), ("mlp.down_proj", 5120, 17408),
)


# ---------------------------------------------------------------- layout ----

def test_selected_tile_divides_every_row_count_exactly() -> None:
    for rows in range(1, 2000):
        tile = select_tile(rows)
        assert rows % tile == 0
        assert tile == (PREFERRED_TILE if rows % PREFERRED_TILE == 0 else rows)


@pytest.mark.parametrize("rows", (0, -1, -256))
def test_selected_tile_rejects_non_positive_rows(rows: int) -> None:
    with pytest.raises(FormatError, match="row count must be positive"):
        select_tile(rows)


@pytest.mark.parametrize(("name", "rows", "columns"), MODEL_TENSOR_SHAPES)
def test_model_tensors_pack_without_padding(name: str, rows: int, columns: int) -> None:
    layout = PackedTensorLayout.for_tensor(rows, columns)
    assert layout.tiles * layout.tile == rows, name
    assert layout.payload_bytes == layout.canonical_bytes
    assert layout.bits_per_weight == pytest.approx(1.75)
    assert layout.codes_shape == (layout.tiles, columns // BLOCK_SIZE, CODE_SLOTS, layout.tile)
    assert layout.canonical_shape == (rows, columns // BLOCK_SIZE, BLOCK_BYTES)


def test_scale_bytes_account_for_the_raw_fp16_scale() -> None:
    assert SCALE_BYTES == 2 and CODE_SLOTS + SCALE_BYTES == BLOCK_BYTES


@pytest.mark.parametrize(
    ("rows", "columns", "tile", "message"),
    ((0, 5120, 256, "dimensions must be positive"), (256, 0, 256, "dimensions must be positive"),
     (256, 5000, 256, "not a multiple"), (256, 5120, 0, "tile must be positive"),
     (100, 5120, 256, "does not divide")),
)
def test_layout_rejects_impossible_geometry(rows, columns, tile, message) -> None:
    with pytest.raises(FormatError, match=message):
        PackedTensorLayout(rows=rows, columns=columns, tile=tile)


def test_layout_json_is_self_describing() -> None:
    payload = PackedTensorLayout.for_tensor(5120, 17408).to_json()
    want = KAT["layout_5120x17408"]
    for key, value in want.items():
        assert payload[key] == value, key
    assert payload["layout_name"] == LAYOUT_NAME


def test_model_census_accounts_for_a_decoded_token() -> None:
    assert sum(s.dispatches_per_token for s in MODEL_LINEAR_SHAPES) == 497


@pytest.mark.parametrize(("rows", "columns"), ((48, 5120), (256, 640), (512, 256), (100, 384), (1024, 384)))
def test_pack_blocks_matches_the_oracle_reorder_and_round_trips(rows: int, columns: int) -> None:
    layout = PackedTensorLayout.for_tensor(rows, columns)
    rng = np.random.default_rng(20260810 + rows + columns)
    blocks = rng.integers(0, 256, size=layout.canonical_shape, dtype=np.uint8)
    codes, scales = pack_blocks(blocks, layout=layout)
    ref_codes, ref_pairs = O.reorder_tensor_arrays(blocks, tile=layout.tile)
    np.testing.assert_array_equal(codes, ref_codes)
    np.testing.assert_array_equal(scales.reshape(-1).view(np.uint8), ref_pairs.reshape(-1))
    assert scales.dtype == np.dtype("<u2") and scales.shape == layout.scales_shape
    np.testing.assert_array_equal(unpack_blocks(codes, scales, layout=layout), blocks)


def test_unpack_rejects_wrong_dtypes_and_shapes() -> None:
    layout = PackedTensorLayout.for_tensor(256, 256)
    codes = np.zeros(layout.codes_shape, dtype=np.uint8)
    scales = np.zeros(layout.scales_shape, dtype="<u2")
    with pytest.raises(FormatError, match="codes must be uint8"):
        unpack_blocks(codes.astype(np.int16), scales, layout=layout)
    with pytest.raises(FormatError, match="little-endian uint16"):
        unpack_blocks(codes, scales.astype(np.int32), layout=layout)
    with pytest.raises(FormatError, match="does not match"):
        unpack_blocks(codes[:, :1], scales, layout=layout)


# ---------------------------------------------------------------- encoder ---

def test_host_encoder_agrees_with_the_oracle_decoder() -> None:
    rng = np.random.default_rng(7)
    scales = rng.integers(0, 256, size=(500, 2), dtype=np.uint8)
    codes = rng.integers(0, 3, size=(500, 128), dtype=np.uint8)
    blocks = encode_tq1_blocks(scales, codes)
    np.testing.assert_array_equal(blocks, O.encode_tq1_blocks(scales, codes))
    got_scales, got_codes = O.decode_tq1_blocks(blocks)
    np.testing.assert_array_equal(got_scales, scales)
    np.testing.assert_array_equal(got_codes, codes)


def test_host_encoder_rejects_non_ternary_codes() -> None:
    codes = np.tile(np.asarray([0, 1, 2, 3], dtype=np.uint8), 32).reshape(1, 128)
    with pytest.raises(FormatError, match="non-ternary"):
        encode_tq1_blocks(np.zeros((1, 2), dtype=np.uint8), codes)


def test_synthetic_distributions() -> None:
    blocks = synthetic.host_blocks(256, 5120, seed=synthetic.SEED_BASE)
    scale_bits, codes = O.decode_tq1_blocks(blocks.reshape(-1, 28))
    fractions = np.bincount(codes.reshape(-1), minlength=3) / codes.size
    np.testing.assert_allclose(fractions, synthetic.TRIT_PROBABILITIES, atol=0.01)
    scales = np.ascontiguousarray(scale_bits).view(np.float16).astype(np.float64).reshape(-1)
    assert scales.min() >= 1e-4 * 0.999
    assert abs(scales.mean() - (0.02 * np.sqrt(2 / np.pi) + 1e-4)) < 1e-3


# -------------------------------------------------------------------- ABI ---

def declared_symbols() -> set[str]:
    header = (ROOT / "include" / "ternel_tq1.h").read_text()
    return set(re.findall(r"\b(ternel_tq1_[a-z_0-9]+)\s*\(", header))


def test_library_exports_every_declared_symbol() -> None:
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    declared = declared_symbols()
    assert declared == set(_lib.SIGNATURES), "the binding and the header list different functions"
    for name in declared:
        assert hasattr(handle, name), name


def test_library_reports_version_and_empty_error() -> None:
    handle = _lib.lib()
    assert handle.ternel_tq1_version().decode().startswith("ternel-tq1-gfx950")
    assert isinstance(handle.ternel_tq1_last_error(), bytes)


def test_argument_errors_are_reported_without_a_launch() -> None:
    """Geometry is checked on the host before any HIP call, with the reference's messages."""
    handle = _lib.lib()
    rc = handle.ternel_tq1_matmul(None, None, None, 1, 256, 5000, 0, 0, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL
    assert "not a multiple of the 128-weight group" in _lib.last_error()
    rc = handle.ternel_tq1_matmul(None, None, None, 1, 256, 5120, 0, 0, 3, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL
    # geometry passes, then the null pointers are refused
    assert "null pointer" in _lib.last_error() or "does not divide" in _lib.last_error()
    rc = handle.ternel_tq1_gemm(None, None, None, 4, 256, 5120, 2, 0, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL and "fp16" in _lib.last_error()
    rc = handle.ternel_tq1_gemm(None, None, None, 4, 256, 5120, 0, 7, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL and "unknown GEMM form 7" in _lib.last_error()
    rc = handle.ternel_tq1_gemm(None, None, None, 65, 256, 5120, 0, 2, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL and "at most 64 activation rows" in _lib.last_error()
    # every GEMM form loads activations 16 bytes at a time
    for form, M, k_split in ((1, 40, 1), (2, 8, 1), (3, 40, 0)):
        rc = handle.ternel_tq1_gemm(ctypes.c_void_p(4096), ctypes.c_void_p(4104), ctypes.c_void_p(8192), M, 256, 5120,
                                    0, form, k_split, None, 0, None)
        assert rc == _lib.TERNEL_TQ1_EINVAL and "16-byte aligned" in _lib.last_error()
    rc = handle.ternel_tq1_get_rows(None, 256, 5120, None, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL and "indices are empty" in _lib.last_error()
    rc = handle.ternel_tq1_get_rows_canonical(ctypes.c_void_p(4098), 256, 5120, None, 1, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL and "4-byte aligned" in _lib.last_error()
    rc = handle.ternel_tq1_get_rows_canonical(ctypes.c_void_p(4096), 256, 5120, None, 0, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL and "indices are empty" in _lib.last_error()


@pytest.mark.parametrize(("M", "rows", "columns", "message"), [
    (1, 0, 5120, "dimensions must be positive"),
    (1, 256, -128, "dimensions must be positive"),
    (0, 256, 5120, "empty batch dimension"),
    (1, 2**31, 5120, "too large for 32-bit"),
    (2**31, 256, 5120, "too large for 32-bit"),
    (1, 256, 128 * (2**31 // 7 + 1), "too large for 32-bit"),
])
def test_geometry_limits_are_refused_before_any_launch(M: int, rows: int, columns: int, message: str) -> None:
    """Sizes past the kernels' 32-bit row, batch and word indices fail with EINVAL on the
    host, for every compute entry point, before any device memory is touched."""
    handle = _lib.lib()
    x = ctypes.c_char_p(b"x" * 16)
    calls = {
        "matmul": lambda: handle.ternel_tq1_matmul(x, x, x, M, rows, columns, 0, 0, 0, None, 0, None),
        "gemm": lambda: handle.ternel_tq1_gemm(x, x, x, M, rows, columns, 0, 0, 0, None, 0, None),
        "linear": lambda: handle.ternel_tq1_linear(x, x, x, M, rows, columns, 0, None, 0, None),
    }
    for name, call in calls.items():
        assert call() == _lib.TERNEL_TQ1_EINVAL, name
        assert message in _lib.last_error(), (name, _lib.last_error())


def test_split_k_refusal_message() -> None:
    handle = _lib.lib()
    x = ctypes.c_char_p(b"x" * 16)
    rc = handle.ternel_tq1_matmul(x, x, x, 1, 256, 5120, 0, 1, 3, None, 0, None)
    assert rc == _lib.TERNEL_TQ1_EINVAL
    assert _lib.last_error() == "k split 3 does not divide the tensor's 40 groups per row"


def test_workspace_queries() -> None:
    handle = _lib.lib()
    # every split workspace: a fixed 64 KiB counter region (its last word the
    # error word), then fp32 partials
    counters = 64 * 1024
    # one vector, strips of at most 96 rows (256 CUs without a GPU) and at most
    # 40 groups: the strip GEMV, which needs no workspace
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 17408, 5120, 0, 0) == 0
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 17408, 5120, 1, 0) == counters + 10 * 17408 * 4
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 8192, 5120, 0, 0) == 0
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 4096, 4096, 0, 0) == 0
    assert handle.ternel_tq1_swiglu_workspace_bytes(1, 12288, 5120, 0) == 0
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 24576, 5120, 0, 0) == 0
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 24578, 5120, 0, 0) > 0  # 98-row strips: LUT23
    # more than 40 groups: the strip GEMV in Z = ceil(G / 40) <= 4 K chunks,
    # whose row partials meet in Z - 1 exchange slots per row of the counter
    # region (so at most 16368 slots); otherwise LUT23
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 8192, 8192, 0, 0) == counters
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 5120, 17408, 0, 0) == counters
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 5120, 17408, 1, 0) == counters + 17 * 5120 * 4
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 5120, 161 * 128, 0, 0) == (
        handle.ternel_tq1_matmul_workspace_bytes(1, 5120, 161 * 128, 1, 0))  # 161 groups: LUT23
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 6144, 17408, 0, 0) == (
        handle.ternel_tq1_matmul_workspace_bytes(1, 6144, 17408, 1, 0))  # 3 x 6144 slots: LUT23
    # the fused SwiGLU form is not split: LUT23 past 40 groups
    assert handle.ternel_tq1_swiglu_workspace_bytes(1, 8192, 8192, 0) == (
        handle.ternel_tq1_matmul_workspace_bytes(1, 8192, 8192, 1, 0))
    assert handle.ternel_tq1_swiglu_workspace_bytes(1, 34816, 5120, 0) == counters + 10 * 34816 * 4
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 256, 5120, 1, 1) == 0
    assert handle.ternel_tq1_matmul_workspace_bytes(1, 256, 5120, 1, 8) == counters + 8 * 256 * 4
    tile, direct = 1, 2
    assert handle.ternel_tq1_gemm_workspace_bytes(512, 17408, 5120, tile, 1) == 0
    assert handle.ternel_tq1_gemm_workspace_bytes(8, 256, 5120, tile, 5) == counters + 5 * 8 * 256 * 4
    # auto: the wide form above 64 rows, the tile form when a K split is fixed
    assert handle.ternel_tq1_gemm_workspace_bytes(512, 17408, 5120, 0, 1) == (
        handle.ternel_tq1_gemm_workspace_bytes(512, 17408, 5120, 3, 1))
    assert handle.ternel_tq1_gemm_workspace_bytes(512, 17408, 5120, 0, 2) == counters + 2 * 512 * 17408 * 4
    # direct form: partials are 128 rows x 32 (or 64) activation columns per row block and chunk
    assert handle.ternel_tq1_gemm_workspace_bytes(8, 256, 5120, direct, 1) == 0
    # partials of the 8 real activation columns only
    assert handle.ternel_tq1_gemm_workspace_bytes(8, 256, 5120, direct, 5) == counters + 5 * 2 * 128 * 8 * 4
    assert handle.ternel_tq1_gemm_workspace_bytes(40, 300, 5120, direct, 4) == counters + 4 * 3 * 128 * 64 * 4
    # auto split: the smallest with chunks of a multiple of 8 groups (of 4 at 17-32 rows) that
    # reaches 512 workgroups -- gate/up 136 row blocks x 5 at any batch, QKV at 32 rows 64 x 10
    assert handle.ternel_tq1_gemm_workspace_bytes(16, 17408, 5120, direct, 0) == counters + 5 * 136 * 128 * 16 * 4
    assert handle.ternel_tq1_gemm_workspace_bytes(32, 17408, 5120, direct, 0) == counters + 5 * 136 * 128 * 32 * 4
    assert handle.ternel_tq1_gemm_workspace_bytes(16, 8192, 5120, direct, 0) == counters + 5 * 64 * 128 * 16 * 4
    assert handle.ternel_tq1_gemm_workspace_bytes(32, 8192, 5120, direct, 0) == counters + 10 * 64 * 128 * 32 * 4
    assert handle.ternel_tq1_gemm_workspace_bytes(65, 256, 5120, direct, 1) == 0  # rejected
    # wide form: two fp32 partial slots of 8 waves x NB fragments x 16 x 64 per
    # workgroup (one per CU, 256 without a GPU, at most one per unit), then
    # the fp16 copy of the activations (K-permuted at four or eight blocks;
    # fp16 x is read in place at one or two, bf16 x always converted into it),
    # then the bf16 rows' inverse scales (M floats, in 256-byte units);
    # NB = 1, 2, 4, 8 32-row activation blocks per tile for M <= 32, 64, 128, above,
    # and 4 instead of 8 while, with 256-wide tiles, the partials a tile's last
    # contributor reads (256/tiles - 1) exceed a tenth of the steps per CU
    # (tiles x groups / 256)
    wide = 3
    def slot_pair(nb: int) -> int:
        return 2 * 8 * nb * 16 * 64 * 4

    def copy(M: int, K: int) -> int:
        return M * K * 2 + (M * 4 + 255) // 256 * 256
    # gate/up, 68 x 2 tiles, 40 groups: 0.9 partials after 21.25 steps
    assert handle.ternel_tq1_gemm_workspace_bytes(512, 17408, 5120, wide, 0) == (
        counters + 256 * slot_pair(8) + copy(512, 5120))
    # gate/up, 68 tiles: 2.8 partials after 10.6 steps
    assert handle.ternel_tq1_gemm_workspace_bytes(256, 17408, 5120, wide, 0) == (
        counters + 256 * slot_pair(4) + copy(256, 5120))
    # down, 20 x 4 tiles, 136 groups: 2.2 partials after 42.5 steps; 20 x 3: 3.3 after 31.9
    assert handle.ternel_tq1_gemm_workspace_bytes(1024, 5120, 17408, wide, 0) == (
        counters + 256 * slot_pair(8) + copy(1024, 17408))
    assert handle.ternel_tq1_gemm_workspace_bytes(768, 5120, 17408, wide, 0) == (
        counters + 256 * slot_pair(4) + copy(768, 17408))
    assert handle.ternel_tq1_gemm_workspace_bytes(5, 256, 640, wide, 1) == counters + 5 * slot_pair(1) + copy(5, 640)
    assert handle.ternel_tq1_gemm_workspace_bytes(64, 17408, 5120, wide, 0) == (
        counters + 256 * slot_pair(2) + copy(64, 5120))
    assert handle.ternel_tq1_gemm_workspace_bytes(100, 17408, 5120, wide, 0) == (
        counters + 256 * slot_pair(4) + copy(100, 5120))
    # bf16 through the library's dispatch: the wide form's workspace
    assert handle.ternel_tq1_linear_workspace_bytes(512, 17408, 5120, 1) == (
        handle.ternel_tq1_gemm_workspace_bytes(512, 17408, 5120, wide, 0))
    assert handle.ternel_tq1_gemm_workspace_bytes(5, 256, 640, wide, 2) == 0  # K is split by stream-K
    assert handle.ternel_tq1_gemm_workspace_bytes(5, 256, 1 << 22, wide, 0) == 0  # 32-bit buffer offsets
    assert handle.ternel_tq1_packed_words(300, 640) == 5 * 5 * 7 * 64
    assert handle.ternel_tq1_packed_words(300, 600) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path) -> None:
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(_lib.NativeLibraryMissing):
        _lib.lib()
