"""GPU decode and fail-closed validation, bit-exact against the oracle and the
closed-form truth table (every byte value, every slot)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.conftest import GOLDEN
from tests.gpu_util import random_blocks, to_dev
from ternel_amd.format import (
    FormatError,
    count_invalid_bytes,
    decode_tq1_blocks,
    validate_blocks,
    validate_packed_codes,
)

pytestmark = pytest.mark.gpu
TRUTH = np.load(GOLDEN / "decode_truth_table.npz")


def test_every_byte_value_in_every_slot_decodes_bit_exactly() -> None:
    blocks = np.zeros((256, 28), dtype=np.uint8)
    blocks[:, 2:28] = np.arange(256, dtype=np.uint8)[:, None]
    blocks[:, 0] = np.arange(256, dtype=np.uint8)
    blocks[:, 1] = 255 - np.arange(256, dtype=np.uint8)
    scales, codes = decode_tq1_blocks(blocks, validate=False)
    np.testing.assert_array_equal(scales, blocks[:, :2])
    regular = codes[:, :125].reshape(256, 25, 5)
    for slot in range(25):
        np.testing.assert_array_equal(regular[:, slot], TRUTH["regular_digits"])
    np.testing.assert_array_equal(codes[:, 125:], TRUTH["tail_digits"])
    ref_scales, ref_codes = O.decode_tq1_blocks(blocks, validate=False)
    np.testing.assert_array_equal(codes, ref_codes)


def test_random_blocks_decode_like_the_oracle() -> None:
    blocks = random_blocks(333, 640, seed=3).reshape(-1, 28)
    got = decode_tq1_blocks(to_dev(blocks))
    want = O.decode_tq1_blocks(blocks)
    np.testing.assert_array_equal(got[0].cpu().numpy(), want[0])
    np.testing.assert_array_equal(got[1].cpu().numpy(), want[1])


def test_all_fp16_scale_patterns_survive_decode() -> None:
    scales = np.arange(1 << 16, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    codes = np.ones((1 << 16, 128), dtype=np.uint8)
    blocks = O.encode_tq1_blocks(scales, codes)
    got_scales, got_codes = decode_tq1_blocks(blocks)
    assert got_scales.tobytes() == scales.tobytes()
    assert (got_codes == 1).all()


@pytest.mark.parametrize(("index", "value", "message"), [
    (2, 243, "invalid base-3 bytes: regular=1, tail=0"),
    (27, 27, "invalid base-3 bytes: regular=0, tail=1"),
])
def test_reference_rejections(index: int, value: int, message: str) -> None:
    blocks = np.zeros((1, 28), dtype=np.uint8)
    blocks[0, index] = value
    with pytest.raises(FormatError) as info:
        decode_tq1_blocks(blocks)
    assert str(info.value) == message


@pytest.mark.parametrize("nblocks", [1, 3, 4, 7, 1000, 65537, 1 << 20])
def test_validation_counts_every_planted_byte(nblocks: int) -> None:
    rng = np.random.default_rng(nblocks)
    blocks = random_blocks(nblocks, 128, seed=nblocks).reshape(-1, 28)
    planted = min(nblocks, 50)
    which = rng.choice(nblocks, size=planted, replace=False)
    for i, b in enumerate(which):
        pos = int(rng.integers(0, 28))
        blocks[b, pos] = 243 + (i % 13) if pos < 27 else 27 + (i % 229)
    want = O.count_invalid(blocks)
    assert count_invalid_bytes(to_dev(blocks)) == want


def test_scale_bytes_are_never_counted() -> None:
    blocks = np.zeros((64, 28), dtype=np.uint8)
    blocks[:, 0:2] = 255
    assert count_invalid_bytes(blocks) == (0, 0)
    validate_blocks(blocks)


def test_load_time_scan_message() -> None:
    blocks = np.zeros((8, 28), dtype=np.uint8)
    blocks[3, 5] = 250
    blocks[4, 27] = 200
    with pytest.raises(FormatError, match=r"out-of-range base-3 bytes: regular=1 \(max 242\), tail=1 \(max 26\)"):
        validate_packed_codes(blocks)


def test_empty_input_validates() -> None:
    assert count_invalid_bytes(torch.zeros((0, 28), dtype=torch.uint8, device="cuda")) == (0, 0)
