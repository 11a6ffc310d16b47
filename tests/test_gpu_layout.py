"""The packed device layout: an exact 4-byte-granularity permutation of the
canonical blocks into 64-row tiles, checked against its index formula restated
here in numpy, and round-tripped."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpu_util import layout, random_blocks, to_dev
from ternel_amd.kernels import pack_weights, packed_shape, unpack_weights

pytestmark = pytest.mark.gpu


def reference_interleave(blocks: np.ndarray) -> np.ndarray:
    """word j of block (r, g) -> packed[r // 64, g, j, r % 64]; padded rows are zero."""
    rows, groups, _ = blocks.shape
    tiles = -(-rows // 64)
    words = np.ascontiguousarray(blocks).view("<u4").reshape(rows, groups, 7)
    out = np.zeros((tiles * 64, groups, 7), dtype=np.uint32)
    out[:rows] = words
    return out.reshape(tiles, 64, groups, 7).transpose(0, 2, 3, 1).copy()


@pytest.mark.parametrize(("rows", "columns"), ((1, 128), (48, 384), (64, 256), (300, 640), (1024, 5120)))
def test_interleave_matches_the_index_formula_and_round_trips(rows: int, columns: int) -> None:
    blocks = np.random.default_rng(rows + columns).integers(0, 256, size=(rows, columns // 128, 28), dtype=np.uint8)
    lay = layout(rows, columns)
    packed = pack_weights(to_dev(blocks.reshape(-1, 28)), layout=lay)
    assert tuple(packed.shape) == packed_shape(lay)
    np.testing.assert_array_equal(packed.cpu().numpy().view(np.uint32), reference_interleave(blocks))
    np.testing.assert_array_equal(unpack_weights(packed, layout=lay).cpu().numpy(), blocks)


def test_packing_preserves_every_byte_value_position() -> None:
    blocks = random_blocks(130, 256, seed=3)
    lay = layout(130, 256)
    back = unpack_weights(pack_weights(to_dev(blocks.reshape(-1, 28)), layout=lay), layout=lay)
    assert back.dtype == torch.uint8
    np.testing.assert_array_equal(back.cpu().numpy(), blocks)
