"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so that a plausible mistake in the oracle fails it: the
golden truth table (pure-Python repeated division), the reference's own
known-answer tests restated as data, exact-integer positional vectors, a
brute-force tiny product, agreement of three independently written products,
and planted mistakes that must be caught.
"""

from __future__ import annotations

import itertools
import json

import numpy as np
import pytest

from oracle import tq1_oracle as O
from tests.conftest import GOLDEN

TRUTH = np.load(GOLDEN / "decode_truth_table.npz")
SMALL = np.load(GOLDEN / "small_product.npz")
KAT = json.loads((GOLDEN / "known_answers.json").read_text())
POWERS = (1, 3, 9, 27, 81)


def all_bytes_blocks() -> np.ndarray:
    """256 blocks: block p carries byte p in every regular slot and in the tail."""
    blocks = np.zeros((256, 28), dtype=np.uint8)
    blocks[:, 2:28] = np.arange(256, dtype=np.uint8)[:, None]
    blocks[:, 0] = 0x00
    blocks[:, 1] = 0x3C  # scale 1.0
    return blocks


# ---------------------------------------------------------------- decode ----

def test_decode_matches_the_closed_form_truth_table_for_every_byte() -> None:
    _, codes = O.decode_tq1_blocks(all_bytes_blocks(), validate=False)
    regular = codes[:, :125].reshape(256, 25, 5)
    for slot in range(25):
        np.testing.assert_array_equal(regular[:, slot, :], TRUTH["regular_digits"])
    np.testing.assert_array_equal(codes[:, 125:], TRUTH["tail_digits"])


def test_count_invalid_matches_the_truth_table_legality() -> None:
    blocks = all_bytes_blocks()
    regular, tail = O.count_invalid(blocks)
    assert regular == 25 * int(np.count_nonzero(~TRUTH["legal_regular"]))
    assert tail == int(np.count_nonzero(~TRUTH["legal_tail"]))


@pytest.mark.parametrize("case", ["reject_regular_243", "reject_tail_27"])
def test_reference_rejection_known_answers(case: str) -> None:
    """tests/test_format.py:105-113: byte 243 -> regular=1, tail 27 -> tail=1."""
    kat = KAT[case]
    blocks = np.zeros((1, 28), dtype=np.uint8)
    blocks[0, kat["byte_index"]] = kat["value"]
    with pytest.raises(O.OracleFormatError) as info:
        O.decode_tq1_blocks(blocks)
    assert str(info.value) == kat["message"]


def test_shape_errors_match_the_reference_messages() -> None:
    with pytest.raises(O.OracleFormatError, match=KAT["shape_messages"]["length"]):
        O.decode_tq1_blocks(np.zeros(27, dtype=np.uint8))
    with pytest.raises(O.OracleFormatError, match="expected TQ1 blocks shaped"):
        O.decode_tq1_blocks(np.zeros((2, 14), dtype=np.uint8))


def test_every_legal_five_trit_byte_round_trips() -> None:
    """tests/test_format.py:46-58."""
    codes = np.ones((243, 128), dtype=np.uint8)
    codes[:, :5] = TRUTH["regular_digits"][:243]
    scales = np.arange(243, dtype=np.uint16).view(np.uint8).reshape(243, 2)
    packed = O.encode_tq1_blocks(scales, codes)
    np.testing.assert_array_equal(packed[:, 2], np.arange(243, dtype=np.uint8))
    got_scales, got_codes = O.decode_tq1_blocks(packed)
    np.testing.assert_array_equal(got_scales, scales)
    np.testing.assert_array_equal(got_codes, codes)


def test_every_legal_tail_byte_round_trips() -> None:
    """tests/test_format.py:61-71."""
    codes = np.ones((27, 128), dtype=np.uint8)
    codes[:, 125:] = TRUTH["tail_digits"][:27]
    packed = O.encode_tq1_blocks(np.tile([[0x34, 0x12]], (27, 1)).astype(np.uint8), codes)
    np.testing.assert_array_equal(packed[:, 27], np.arange(27, dtype=np.uint8))
    np.testing.assert_array_equal(O.decode_tq1_blocks(packed)[1], codes)


def test_all_fp16_scale_bit_patterns_survive() -> None:
    """tests/test_format.py:84-91."""
    scales = np.arange(1 << 16, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    codes = np.ones((1 << 16, 128), dtype=np.uint8)
    got, _ = O.decode_tq1_blocks(O.encode_tq1_blocks(scales, codes))
    assert got.tobytes() == scales.tobytes()


def test_all_ternary_patterns_round_trip() -> None:
    """tests/test_format.py:74-81."""
    patterns = np.asarray(list(itertools.product(range(3), repeat=5)), dtype=np.uint8)
    codes = np.resize(patterns.reshape(-1), 4 * 128).reshape(4, 128)
    scales = np.asarray([[0, 0], [0, 0x80], [0, 0x7C], [0xFF, 0x7B]], dtype=np.uint8)
    got_scales, got_codes = O.decode_tq1_blocks(O.encode_tq1_blocks(scales, codes))
    np.testing.assert_array_equal(got_scales, scales)
    np.testing.assert_array_equal(got_codes, codes)


def test_encode_rejects_non_ternary_codes() -> None:
    codes = np.zeros((1, 128), dtype=np.uint8)
    codes[0, 7] = 3
    with pytest.raises(O.OracleFormatError, match="non-ternary"):
        O.encode_tq1_blocks(np.zeros((1, 2), dtype=np.uint8), codes)


def test_lut23_split_is_exact_for_every_legal_byte() -> None:
    """tests/test_format.py:351-357: (p*57)>>9 == p//9 for p <= 242 (and up to 511)."""
    for p in range(256):
        hi = (p * 57) >> 9
        assert (hi, p - 9 * hi) == tuple(TRUTH["lut23_split"][p]) or p > 242
    assert all(((p * 57) >> 9) == p // 9 for p in range(512))


# ---------------------------------------------------------------- layout ----

@pytest.mark.parametrize("rows", (1, 48, 256, 257, 513))
def test_reorder_index_formula_and_round_trip(rows: int) -> None:
    """lut23_reorder.py:140-141 index formula, brute-forced; tests/test_format.py:292-307 round trip."""
    rng = np.random.default_rng(20260809 + rows)
    blocks = rng.integers(0, 256, size=(rows, 3, 28), dtype=np.uint8)
    codes, scales = O.reorder_tensor_arrays(blocks, tile=256)
    for r in range(0, rows, max(1, rows // 7)):
        for g in range(3):
            for s in range(26):
                assert codes[r // 256, g, s, r % 256] == blocks[r, g, 2 + s]
            assert tuple(scales[r // 256, g, r % 256]) == tuple(blocks[r, g, :2])
    np.testing.assert_array_equal(O.restore_tensor_arrays(codes, scales, rows, tile=256), blocks)
    padded = codes.shape[-1] - (rows % 256 or 256)
    if padded:
        assert not codes[-1, :, :, -padded:].any()


# -------------------------------------------------------------- products ----

def _positional_case(slot: int | None):
    """All 243 legal bytes in one slot (or all 27 tail bytes), scale 1, positional x."""
    if slot is None:
        rows = 27
        blocks = np.zeros((rows, 28), dtype=np.uint8)
        blocks[:, 2:27] = 121  # neutral: all trits 1 -> weight 0
        blocks[:, 27] = np.arange(27)
        x = np.zeros((1, 128), dtype=np.float32)
        x[0, 125:128] = POWERS[:3]
        want = TRUTH["positional_tail"][:27]
    else:
        rows = 243
        blocks = np.zeros((rows, 28), dtype=np.uint8)
        blocks[:, 2:27] = 121
        blocks[:, 27] = 13
        blocks[:, 2 + slot] = np.arange(243)
        x = np.zeros((1, 128), dtype=np.float32)
        x[0, 5 * slot:5 * slot + 5] = POWERS
        want = TRUTH["positional_regular"][:243]
    blocks[:, 0], blocks[:, 1] = 0x00, 0x3C
    return blocks.reshape(rows, 1, 28), x, want.astype(np.float64)


@pytest.mark.parametrize("slot", [0, 7, 24, None])
@pytest.mark.parametrize("product", ["reference_gemv", "lut23_matmul", "oracle_matmul", "cpu_decode_matmul"])
def test_positional_vectors_give_exact_integers(slot, product: str) -> None:
    """tests/test_mlx_kernels.py:107-153 pattern: byte - 121 per slot, byte - 13 for the tail."""
    blocks, x, want = _positional_case(slot)
    rows = blocks.shape[0]
    if product == "reference_gemv":
        got = O.reference_gemv(blocks, x[0], rows=rows, columns=128)
    else:
        got = getattr(O, product)(blocks, x, rows=rows, columns=128)[0]
    np.testing.assert_array_equal(np.asarray(got, dtype=np.float64), want)


@pytest.mark.parametrize("product", ["reference_gemv", "lut23_matmul", "oracle_matmul", "cpu_decode_matmul"])
def test_small_brute_force_product(product: str) -> None:
    blocks, x, want = SMALL["blocks"], SMALL["x"], SMALL["expected"]
    if product == "reference_gemv":
        got = O.reference_gemv(blocks, x[0], rows=3, columns=256)[None]
    else:
        got = getattr(O, product)(blocks, x, rows=3, columns=256)
    np.testing.assert_array_equal(np.asarray(got, dtype=np.float64), want)


def test_dense_weights_match_the_brute_force_trits() -> None:
    w = O.dense_weights(SMALL["blocks"], rows=3, columns=256)
    scales = np.array([0.5, 1.0, 2.0, 0.25, 4.0, 0.125]).reshape(6, 1)
    want = ((SMALL["trits"].astype(np.float64) - 1.0) * scales).reshape(3, 256)
    np.testing.assert_array_equal(w, want)


def test_three_products_agree_within_fp32_rounding() -> None:
    """tests/test_mlx_kernels.py:230-243: all within 1e-6 of the fp64 oracle."""
    rng = np.random.default_rng(5)
    rows, columns = 96, 640
    scales = rng.normal(0, 0.05, size=rows * 5).astype(np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(rows * 5, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, trits).reshape(rows, 5, 28)
    x = rng.normal(0, 1, size=(3, columns)).astype(np.float32)
    oracle = O.oracle_matmul(blocks, x, rows=rows, columns=columns)
    lut = O.lut23_matmul(blocks, x, rows=rows, columns=columns)
    ref = np.stack([O.reference_gemv(blocks, x[i], rows=rows, columns=columns) for i in range(3)])
    for got in (lut, ref):
        assert O.compare(got, oracle)["normalised_max_abs_error"] < 1e-6
    # the CPU baseline arm rounds its fp32 product to fp16 once
    cpu = O.cpu_decode_matmul(blocks, x, rows=rows, columns=columns).astype(np.float64)
    assert np.all(np.abs(cpu - oracle) <= np.abs(oracle) * 2.0**-11 + 1e-6 * np.abs(oracle).max())


def test_get_rows_reference_closed_form() -> None:
    blocks = SMALL["blocks"]
    got = O.get_rows_reference(blocks, [2, 0, 5, -1], rows=3, columns=256)
    w = O.dense_weights(blocks, rows=3, columns=256).astype(np.float32)
    np.testing.assert_array_equal(got[0], w[2])
    np.testing.assert_array_equal(got[1], w[0])
    assert not got[2].any() and not got[3].any()
    with pytest.raises(O.OracleFormatError, match="outside"):
        O.get_rows_reference(blocks, [3], rows=3, columns=256, out_of_range="raise")


# ------------------------------------------------------------ comparator ----

def test_compare_catches_a_relocated_nan_and_a_sign_flipped_inf() -> None:
    """kernel_gate.py:275-287 semantics (tests/test_mlx_kernel_gate.py:88-139)."""
    want = np.array([[1.0, np.nan, 3.0], [np.inf, 1.0, 2.0]])
    moved = np.array([[np.nan, 1.0, 3.0], [np.inf, 1.0, 2.0]])
    flipped = np.array([[1.0, np.nan, 3.0], [-np.inf, 1.0, 2.0]])
    assert O.compare(want, want)["bit_exact"]
    assert O.compare(moved, want)["pattern_mismatches"] == 2
    assert O.compare(flipped, want)["pattern_mismatches"] == 1


def test_compare_normalises_per_case() -> None:
    """A huge case cannot excuse a wrong small one (tests/test_mlx_kernel_gate.py:34)."""
    want = np.array([[1e18, 2e18], [1.0, 2.0]])
    got = np.array([[1e18, 2e18], [1.5, 2.0]])
    assert O.compare(got, want)["normalised_max_abs_error"] == pytest.approx(0.25)


# ------------------------------------------------------ planted mistakes ----

def test_a_swapped_trit_decoder_fails_the_positional_vectors() -> None:
    """Plant a mistake in a copy of the oracle's decoder and require the KAT to catch it."""
    blocks, x, want = _positional_case(3)

    def broken_dense(b, *, rows, columns, dtype=np.float64):
        w = O.dense_weights(b, rows=rows, columns=columns, dtype=dtype).reshape(rows, -1, 128)
        w[:, :, [15, 16]] = w[:, :, [16, 15]]  # swap trits 0 and 1 of slot 3
        return w.reshape(rows, columns)

    got = (x.astype(np.float64) @ broken_dense(blocks, rows=243, columns=128).T)[0]
    assert not np.array_equal(got, want)


def test_a_dropped_tail_fails_the_tail_vector() -> None:
    blocks, x, want = _positional_case(None)
    w = O.dense_weights(blocks, rows=27, columns=128)
    w[:, 125:] = 0.0
    assert not np.array_equal((x.astype(np.float64) @ w.T)[0], want)


def test_an_off_by_one_lut_split_fails_the_truth_table() -> None:
    bad = [((p * 57) >> 8, p - 9 * ((p * 57) >> 8)) for p in range(243)]
    assert any(tuple(TRUTH["lut23_split"][p]) != bad[p] for p in range(243))


def q2_pack_python(scales: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """Bit-by-bit Q2_0 packer: quant byte j holds codes 4j..4j+3, code 4j+k in bits 2k, 2k+1."""
    out = np.zeros((codes.shape[0], 34), dtype=np.uint8)
    for n in range(codes.shape[0]):
        out[n, 0:2] = scales[n]
        for j in range(32):
            byte = 0
            for k in range(4):
                byte |= int(codes[n, 4 * j + k]) << (2 * k)
            out[n, 2 + j] = byte
    return out


def test_q2_decoder_order_known_answer() -> None:
    """tests/test_format.py:94-102: codes 0,1,2,3 repeated, scale bytes 0xAA 0x55."""
    codes = np.tile(np.asarray([0, 1, 2, 3], dtype=np.uint8), 32).reshape(1, 128)
    scales = np.asarray([[0xAA, 0x55]], dtype=np.uint8)
    source = q2_pack_python(scales, codes)
    assert source[0, 2] == 0b11100100
    got_scales, got_codes = O.decode_q2_blocks(source)
    np.testing.assert_array_equal(got_scales, scales)
    np.testing.assert_array_equal(got_codes, codes)


def test_q2_decoder_matches_bit_extraction_for_every_byte_value() -> None:
    source = np.zeros((256, 34), dtype=np.uint8)
    source[:, 2:] = np.arange(256, dtype=np.uint8)[:, None]
    source[:, 2 + 5] = np.arange(256, dtype=np.uint8)[::-1]  # a different value at one position
    _, codes = O.decode_q2_blocks(source)
    for v in range(256):
        for j in range(32):
            byte = 255 - v if j == 5 else v
            assert [int(c) for c in codes[v, 4 * j:4 * j + 4]] == [(byte >> (2 * k)) & 3 for k in range(4)]


def test_q2_and_tq1_dense_weights_agree_after_repacking() -> None:
    """tests/test_format.py:146-158: the Q2 source and its TQ1 re-encoding are the same matrix."""
    rng = np.random.default_rng(20260808)
    rows, columns = 3, 256
    groups = rows * columns // 128
    scales = rng.integers(1, 0x7BFF, size=groups, dtype=np.uint16).view(np.uint8).reshape(groups, 2)
    codes = rng.integers(0, 3, size=(groups, 128), dtype=np.uint8)
    source = q2_pack_python(scales, codes)
    packed = O.encode_tq1_blocks(*O.decode_q2_blocks(source))
    np.testing.assert_array_equal(O.q2_dense_weights(source, rows=rows, columns=columns),
                                  O.dense_weights(packed.reshape(rows, -1, 28), rows=rows, columns=columns))
    x = rng.normal(size=columns).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(O.reference_gemv(packed, x, rows=rows, columns=columns),
                                  O.reference_gemv(O.encode_tq1_blocks(scales, codes), x, rows=rows, columns=columns))
