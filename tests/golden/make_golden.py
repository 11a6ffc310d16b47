"""Write the committed golden fixtures for the TQ1_G128 path.

Everything here is computed from first principles with pure-Python integers --
repeated division by 3, explicit loops -- deliberately sharing no code with
``oracle/tq1_oracle.py`` or ``ternel_amd``, so that the fixtures pin both of
them. No reference code is imported or run: the known-answer values below are
the ones the reference's own tests assert (tests/test_format.py,
tests/test_mlx_kernels.py), restated as data.

Run: ``python tests/golden/make_golden.py`` (rewrites the .npz files beside it).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def truth_table() -> dict[str, np.ndarray]:
    """For every byte 0..255: its five base-3 digits (regular slot), three (tail),
    legality in either position, and the LUT23 split (p // 9, p % 9).

    Digits are ``(p // 3**i) % 3`` -- for illegal bytes the top digit of a
    regular slot is ``(p // 81) % 3``, which is what format.py:114-118 computes.
    """
    regular = np.zeros((256, 5), dtype=np.uint8)
    tail = np.zeros((256, 3), dtype=np.uint8)
    for p in range(256):
        q = p
        for i in range(5):
            regular[p, i] = q % 3
            q //= 3
        tail[p] = regular[p, :3]
        # explicit cross-check of the repeated-division form against powers
        assert [int(v) for v in regular[p]] == [(p // 3**i) % 3 for i in range(5)]
    legal_regular = np.array([p <= 242 for p in range(256)], dtype=bool)
    legal_tail = np.array([p <= 26 for p in range(256)], dtype=bool)
    split = np.array([[p // 9, p % 9] for p in range(256)], dtype=np.int32)
    # Positional value sum_i (t_i - 1) * 3**i of a regular byte = p - 121; tail = p - 13.
    positional_regular = np.array([sum((int(d) - 1) * 3**i for i, d in enumerate(regular[p])) for p in range(256)],
                                  dtype=np.int32)
    positional_tail = np.array([sum((int(d) - 1) * 3**i for i, d in enumerate(tail[p])) for p in range(256)],
                               dtype=np.int32)
    return {
        "regular_digits": regular,
        "tail_digits": tail,
        "legal_regular": legal_regular,
        "legal_tail": legal_tail,
        "lut23_split": split,
        "positional_regular": positional_regular,
        "positional_tail": positional_tail,
    }


def small_product_vectors() -> dict[str, np.ndarray]:
    """Tiny brute-force products: rows=3, columns=256 (two groups), computed with
    Python integers/floats element by element.

    Scales are powers of two and activations small integers, so every product and
    every partial sum is exact in fp32 and fp64 alike: the expected output is the
    one true answer, independent of summation order.
    """
    rows, groups = 3, 2
    columns = groups * 128
    state = 20261201
    trits = []
    for _ in range(rows * groups * 128):
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        trits.append((state >> 33) % 3)
    scale_values = [0.5, 1.0, 2.0, 0.25, 4.0, 0.125]  # one per (row, group)
    scale_bits = np.array(scale_values, dtype=np.float16).view(np.uint16)
    blocks = np.zeros((rows * groups, 28), dtype=np.uint8)
    for b in range(rows * groups):
        t = trits[b * 128:(b + 1) * 128]
        blocks[b, 0] = int(scale_bits[b]) & 0xFF
        blocks[b, 1] = int(scale_bits[b]) >> 8
        for j in range(25):
            blocks[b, 2 + j] = sum(t[5 * j + i] * 3**i for i in range(5))
        blocks[b, 27] = sum(t[125 + i] * 3**i for i in range(3))
    xs = []
    for k in range(columns):
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        xs.append(float(int((state >> 40) % 9) - 4))
    expected = []
    for r in range(rows):
        total = 0.0
        for g in range(groups):
            b = r * groups + g
            for k in range(128):
                total += (trits[b * 128 + k] - 1) * scale_values[b] * xs[g * 128 + k]
        expected.append(total)
    return {
        "blocks": blocks.reshape(rows, groups, 28),
        "trits": np.array(trits, dtype=np.uint8).reshape(rows * groups, 128),
        "x": np.array(xs, dtype=np.float32).reshape(1, columns),
        "expected": np.array(expected, dtype=np.float64).reshape(1, rows),
    }


def known_answers() -> dict:
    """Assertions of the reference's tests, as data."""
    return {
        # tests/test_format.py:105-113
        "reject_regular_243": {"byte_index": 2, "value": 243, "message": "invalid base-3 bytes: regular=1, tail=0"},
        "reject_tail_27": {"byte_index": 27, "value": 27, "message": "invalid base-3 bytes: regular=0, tail=1"},
        # tests/test_format.py:290-296
        "shape_messages": {
            "length": "TQ1 byte length is not divisible by 28",
            "shape_prefix": "expected TQ1 blocks shaped (N, 28), got",
        },
        # tests/test_mlx_format.py:118-126 (layout JSON for 5120x17408 in the reference's row/column convention)
        "layout_5120x17408": {"tile": 256, "tiles": 20, "groups_per_row": 136, "groups": 5120 * 136,
                              "payload_bytes": 5120 * 136 * 28, "layout_name": "TQ1_G128_MLX_TILED"},
    }


def main() -> None:
    np.savez_compressed(HERE / "decode_truth_table.npz", **truth_table())
    np.savez_compressed(HERE / "small_product.npz", **small_product_vectors())
    (HERE / "known_answers.json").write_text(json.dumps(known_answers(), indent=2, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
