"""Device memory held for a packed weight: one copy per weight.

The reference keeps one array pair per tensor (src/ternel_mlx/modules.py:472-473,
516-517). Here a module keeps its packed words and derives codes/scales on
access; the functional calls' word cache gives up a pair's words as soon as the
pair dies. Also: reloading a module three times leaves its state dict equal to
the last pair loaded, and MFMA-path activations at an unaligned storage offset
are realigned rather than refused.
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from ternel_amd import kernels
from ternel_amd.kernels import GemmConfig, tiled_from_words, tq1_gemm_words, tq1_matmul
from ternel_amd.modules import PackedLinear

from tests.gpu_util import layout, pack, random_blocks, to_dev

pytestmark = pytest.mark.gpu


def _settle() -> int:
    gc.collect()
    torch.cuda.synchronize()
    return torch.cuda.memory_allocated()


def test_a_dead_pair_releases_its_cached_words() -> None:
    rows, columns = 4096, 5120
    lay = layout(rows, columns)
    codes, scales = tiled_from_words(pack(random_blocks(rows, columns, seed=3)), layout=lay)
    x = torch.randn(1, columns, device="cuda", dtype=torch.float16)
    base = _settle()
    tq1_matmul(codes, scales, x, groups_per_row=lay.groups_per_row, tile=lay.tile)
    held = kernels.word_cache_bytes()
    assert held >= rows * (columns // 128) * 28
    del codes, scales
    after = _settle()
    assert kernels.word_cache_bytes() == held - rows * (columns // 128) * 28
    # the pair (codes + scales) and its words are gone; the output and the
    # workspace of the call may remain
    assert after <= base - rows * (columns // 128) * 28 + (8 << 20)


def test_state_dict_keeps_no_second_copy_and_follows_the_last_load() -> None:
    rows, columns = 2048, 5120
    module = PackedLinear(layout(rows, columns))
    pairs = []
    for seed in (11, 12, 13):
        blocks = random_blocks(rows, columns, seed=seed)
        codes, scales = tiled_from_words(pack(blocks), layout=module.layout)
        pairs.append((codes.cpu(), scales.cpu()))
        module.load_weights([("codes", codes), ("scales", scales)])
        del codes, scales
    base = _settle()
    state = module.state_dict()
    np.testing.assert_array_equal(state["codes"].cpu().numpy(), pairs[-1][0].numpy())
    np.testing.assert_array_equal(state["scales"].cpu().numpy(), pairs[-1][1].numpy())
    del state
    assert _settle() <= base
    codes = module.codes
    np.testing.assert_array_equal(codes.cpu().numpy(), pairs[-1][0].numpy())
    del codes
    assert _settle() <= base


def test_unaligned_activation_views_are_realigned_for_the_mfma_forms() -> None:
    rows, columns, batch = 512, 1024, 16
    blocks = random_blocks(rows, columns, seed=5)
    x = np.random.default_rng(5).normal(0, 1, size=(batch, columns)).astype(np.float16)
    storage = torch.zeros(batch * columns + 8, dtype=torch.float16, device="cuda")
    view = storage[3:3 + batch * columns].view(batch, columns)
    view.copy_(to_dev(x))
    assert view.data_ptr() % 16 != 0
    got = tq1_gemm_words(pack(blocks), view, layout=layout(rows, columns), config=GemmConfig())
    oracle = O.oracle_matmul(blocks, x.astype(np.float32), rows=rows, columns=columns)
    assert O.compare(got.float().cpu().numpy(), oracle)["normalised_max_abs_error"] < 1e-3
