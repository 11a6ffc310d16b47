"""Shared helpers for the GPU parity tests (inputs are built on the host with
numpy, uploaded, run through the C ABI, and checked against the CPU oracle)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import tq1_oracle as O
from ternel_amd.layout import PackedTensorLayout

POWERS = (1, 3, 9, 27, 81)


def dev() -> torch.device:
    return torch.device("cuda", 0)


def random_blocks(rows: int, columns: int, seed: int, *, scale_sigma: float = 0.05) -> np.ndarray:
    """Canonical blocks with i.i.d. uniform trits and N(0, sigma) fp16 scales
    (the reference kernel tests' generator, tests/test_mlx_kernels.py:85-95)."""
    rng = np.random.default_rng(seed)
    groups = rows * (columns // 128)
    scales = rng.normal(0.0, scale_sigma, size=groups).astype(np.float16).view(np.uint8).reshape(-1, 2)
    trits = rng.integers(0, 3, size=(groups, 128), dtype=np.uint8)
    return O.encode_tq1_blocks(scales, trits).reshape(rows, columns // 128, 28)


def to_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def layout(rows: int, columns: int) -> PackedTensorLayout:
    return PackedTensorLayout.for_tensor(rows, columns)


def pack(blocks: np.ndarray) -> torch.Tensor:
    """Canonical (rows, G, 28) host blocks -> packed device words."""
    from ternel_amd.kernels import pack_weights

    rows, g, _ = blocks.shape
    return pack_weights(to_dev(blocks.reshape(-1, 28)), layout=layout(rows, g * 128))


def positional_all_slots() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """tests/test_mlx_kernels.py:107-135 construction: 243 rows x 25 groups; group g
    carries the byte under test in slot g; batch sample g has activation
    [1,3,9,27,81] in slot g of group g only. Output[g][p] = p - 121 exactly."""
    rows, groups = 243, 25
    blocks = np.zeros((rows, groups, 28), dtype=np.uint8)
    blocks[:, :, 0], blocks[:, :, 1] = 0x00, 0x3C  # scale 1.0
    blocks[:, :, 2:27] = 121                       # neutral bytes: weight 0
    blocks[:, :, 27] = 13
    for g in range(groups):
        blocks[:, g, 2 + g] = np.arange(rows)
    x = np.zeros((groups, groups * 128), dtype=np.float32)
    for g in range(groups):
        x[g, g * 128 + 5 * g: g * 128 + 5 * g + 5] = POWERS
    want = np.tile(np.arange(rows, dtype=np.float64) - 121.0, (groups, 1))
    return blocks, x, want


def positional_tail() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    rows = 27
    blocks = np.zeros((rows, 1, 28), dtype=np.uint8)
    blocks[:, 0, 0], blocks[:, 0, 1] = 0x00, 0x3C
    blocks[:, 0, 2:27] = 121
    blocks[:, 0, 27] = np.arange(rows)
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, 125:128] = POWERS[:3]
    want = (np.arange(rows, dtype=np.float64) - 13.0)[None]
    return blocks, x, want
