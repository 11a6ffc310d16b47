"""On-device Q2_0 -> TQ1_G128 re-encode against decode_q2_blocks + encode_tq1_blocks."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, to_dev
from ternel_amd.format import FormatError, convert_q2_blocks
from ternel_amd.kernels import tq1_matmul_words

pytestmark = pytest.mark.gpu


def legal_q2(n: int, seed: int, *, scale_bits=None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 3, size=(n, 128), dtype=np.uint8)
    scales = (rng.integers(0, 1 << 16, size=n, dtype=np.uint16) if scale_bits is None else scale_bits)
    scales = scales.astype(np.uint16).view(np.uint8).reshape(n, 2)
    quant = codes.reshape(n, 32, 4).astype(np.uint8)
    source = np.empty((n, 34), dtype=np.uint8)
    source[:, :2] = scales
    source[:, 2:] = quant[:, :, 0] | (quant[:, :, 1] << 2) | (quant[:, :, 2] << 4) | (quant[:, :, 3] << 6)
    return source, scales, codes


@pytest.mark.parametrize("n", (1, 7, 1000, 100003))
def test_conversion_is_bit_exact(n: int) -> None:
    source, scales, codes = legal_q2(n, seed=n)
    want = O.encode_tq1_blocks(*O.decode_q2_blocks(source))
    np.testing.assert_array_equal(want, O.encode_tq1_blocks(scales, codes))
    np.testing.assert_array_equal(convert_q2_blocks(source), want)


def test_every_legal_quant_byte_at_every_position() -> None:
    legal = np.asarray([a | (b << 2) | (c << 4) | (d << 6) for a in range(3) for b in range(3)
                        for c in range(3) for d in range(3)], dtype=np.uint8)  # 81 values
    source, _, _ = legal_q2(32 * 81, seed=3)
    for j in range(32):
        source[j * 81:(j + 1) * 81, 2 + j] = legal
    np.testing.assert_array_equal(convert_q2_blocks(source), O.encode_tq1_blocks(*O.decode_q2_blocks(source)))


def test_every_scale_bit_pattern_is_copied() -> None:
    source, _, _ = legal_q2(1 << 16, seed=4, scale_bits=np.arange(1 << 16, dtype=np.uint16))
    out = convert_q2_blocks(source)
    np.testing.assert_array_equal(out[:, :2], source[:, :2])


@pytest.mark.parametrize("planted", (1, 37))
def test_a_code_of_three_rejects_the_source(planted: int) -> None:
    source, _, _ = legal_q2(500, seed=planted)
    rng = np.random.default_rng(planted)
    for block, code in zip(rng.choice(500, size=planted, replace=False), rng.integers(0, 128, size=planted)):
        source[block, 2 + code // 4] |= 3 << (2 * (code % 4))
    assert int((O.decode_q2_blocks(source)[1] == 3).sum()) == planted
    with pytest.raises(FormatError, match=f"source contains {planted} non-ternary code"):
        convert_q2_blocks(source)


def test_shape_errors_match_the_reference_messages() -> None:
    with pytest.raises(FormatError, match="divisible by 34"):
        convert_q2_blocks(np.zeros(33, dtype=np.uint8))
    with pytest.raises(FormatError, match="expected Q2"):
        convert_q2_blocks(np.zeros((1, 2, 17), dtype=np.uint8))


def test_device_input_stays_on_the_device_and_products_agree() -> None:
    rows, columns = 512, 1024
    source, _, _ = legal_q2(rows * columns // 128, seed=9, scale_bits=np.full(rows * 8, 0x2E66, dtype=np.uint16))
    out = convert_q2_blocks(torch.from_numpy(source).cuda())
    assert out.is_cuda and out.shape == (rows * columns // 128, 28)
    blocks = out.cpu().numpy().reshape(rows, columns // 128, 28)
    x = np.random.default_rng(9).normal(0, 1, size=(2, columns)).astype(np.float32)
    got = tq1_matmul_words(pack(blocks), to_dev(x), layout=layout(rows, columns)).cpu().numpy()
    want = x.astype(np.float64) @ O.q2_dense_weights(source, rows=rows, columns=columns).T
    assert O.compare(got, want)["normalised_max_abs_error"] < 1e-5
