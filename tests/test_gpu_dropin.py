"""The reference's call sequences, replayed against the engine unchanged except
for the array type (torch device tensors for mlx arrays).

Module path (tests/test_mlx_modules.py:116-136, 1114-1234): build a tiled
``codes``/``scales`` pair through the block encoder and ``pack_blocks``,
construct ``PackedLinear(layout)`` / ``PackedEmbedding(layout, dtype=)``, load
with ``load_weights([("codes", c), ("scales", s)])``, call, ``as_linear``.
Functional path (src/ternel_mlx/kernels.py:1215, 1287, 1360; modules.py:425):
``tq1_matmul(codes, scales, x, *, groups_per_row, tile, config)``,
``tq1_gemm(...)``, ``tq1_get_rows(codes, scales, indices, *, groups_per_row,
tile, dtype, threads, safe_clamp)``, ``packed_matmul(codes, scales, x, *,
layout)``. State: ``state_dict`` keys ``codes``/``scales`` and
``load_state_dict`` of artifact-shaped tensors
(tests/test_mlx_modules.py:200-262).

Pinned by the fp64 oracle at the reference's oracle tolerance (1e-5, fp32
activations), the LUT23 oracle bit for bit where the reference holds its
unsplit arm to it, and the closed-form gather.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import tq1_oracle as O
from ternel_amd.format import BLOCK_SIZE, FormatError, encode_tq1_blocks
from ternel_amd.kernels import GemmConfig, MatmulConfig, tq1_gemm, tq1_get_rows, tq1_matmul, words_of
from ternel_amd.layout import PackedTensorLayout, pack_blocks, unpack_blocks
from ternel_amd.modules import PackedEmbedding, PackedLinear, packed_matmul

pytestmark = pytest.mark.gpu

ORACLE_RELATIVE_TOLERANCE = 1e-5  # src/ternel_mlx/kernel_gate.py:105


def random_packed(rows: int, columns: int, seed: int):
    """tests/test_mlx_modules.py:116-129: encoded through the block encoder, then tiled."""
    layout = PackedTensorLayout.for_tensor(rows, columns)
    generator = np.random.default_rng(seed)
    scale_bits = generator.normal(0.0, 0.05, size=layout.groups).astype(np.float16).view(np.uint8).reshape(-1, 2)
    trits = generator.integers(0, 3, size=(layout.groups, BLOCK_SIZE), dtype=np.uint8)
    blocks = encode_tq1_blocks(scale_bits, trits).reshape(rows, layout.groups_per_row, -1)
    codes, scales = pack_blocks(blocks, layout=layout)
    return layout, codes, scales


def device_pair(codes: np.ndarray, scales: np.ndarray) -> tuple[torch.Tensor, torch.Tensor]:
    return torch.from_numpy(codes).cuda(), torch.from_numpy(scales.astype("<u2")).cuda()


def load_packed(module, codes: np.ndarray, scales: np.ndarray) -> None:
    c, s = device_pair(codes, scales)
    module.load_weights([("codes", c), ("scales", s)])


def blocks_of(layout: PackedTensorLayout, codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    return unpack_blocks(codes, scales, layout=layout)


@pytest.mark.parametrize(("rows", "batch"), ((1024, 1), (1024, 2), (1024, 4), (1024, 16), (17408, 16),
                                             (1024, 128), (1024, 188)))
def test_a_packed_linear_matches_the_oracle_across_every_dispatch_regime(rows: int, batch: int) -> None:
    columns = 2 * BLOCK_SIZE
    layout, codes, scales = random_packed(rows, columns, seed=20260810 + batch)
    module = PackedLinear(layout)
    load_packed(module, codes, scales)
    x = np.random.default_rng(4242 + batch).normal(0.0, 1.0, size=(batch, columns)).astype(np.float32)
    out = module(torch.from_numpy(x).cuda()).cpu().numpy()
    assert out.shape == (batch, rows) and np.isfinite(out).all()
    result = O.compare(out, O.oracle_matmul(blocks_of(layout, codes, scales), x, rows=rows, columns=columns))
    assert result["normalised_max_abs_error"] <= ORACLE_RELATIVE_TOLERANCE, result


def test_a_packed_linear_keeps_the_leading_dimensions_of_its_input() -> None:
    rows, columns = 256, BLOCK_SIZE
    layout, codes, scales = random_packed(rows, columns, seed=77)
    module = PackedLinear(layout)
    load_packed(module, codes, scales)
    x = torch.from_numpy(np.random.default_rng(77).normal(0, 1, size=(2, 3, columns)).astype(np.float32)).cuda()
    out = module(x)
    assert tuple(out.shape) == (2, 3, rows)
    np.testing.assert_array_equal(out.reshape(-1, rows).cpu().numpy(), module(x.reshape(-1, columns)).cpu().numpy())


def test_a_packed_embedding_gathers_the_rows_the_reference_does() -> None:
    rows, columns = 512, 2 * BLOCK_SIZE
    layout, codes, scales = random_packed(rows, columns, seed=909)
    module = PackedEmbedding(layout, dtype=torch.float32)
    load_packed(module, codes, scales)
    tokens = np.array([[0, 1, 255, 256], [rows - 1, 7, 128, 42]], dtype=np.int32)
    out = module(torch.from_numpy(tokens).cuda())
    assert tuple(out.shape) == (2, 4, columns)
    want = O.get_rows_reference(blocks_of(layout, codes, scales), tokens.reshape(-1), rows=rows, columns=columns)
    np.testing.assert_array_equal(out.reshape(-1, columns).cpu().numpy(), want)


def test_a_packed_embedding_used_as_a_head_agrees_with_a_packed_linear() -> None:
    rows, columns = 256, BLOCK_SIZE
    layout, codes, scales = random_packed(rows, columns, seed=31337)
    embedding = PackedEmbedding(layout, dtype=torch.float32)
    linear = PackedLinear(layout)
    load_packed(embedding, codes, scales)
    load_packed(linear, codes, scales)
    x = torch.from_numpy(np.random.default_rng(31337).normal(0, 1, size=(4, columns)).astype(np.float32)).cuda()
    np.testing.assert_array_equal(embedding.as_linear(x).cpu().numpy(), linear(x).cpu().numpy())


def test_an_out_of_range_token_id_reads_zero_rather_than_out_of_bounds() -> None:
    rows, columns = 256, BLOCK_SIZE
    layout, codes, scales = random_packed(rows, columns, seed=5)
    module = PackedEmbedding(layout, dtype=torch.float32)
    load_packed(module, codes, scales)
    out = module(torch.tensor([rows, rows + 1000, 0], dtype=torch.int64).cuda()).cpu().numpy()
    assert not out[0].any() and not out[1].any() and out[2].any()


def test_the_canonical_row_copy_is_opt_in_and_gathers_the_same_rows() -> None:
    rows, columns = 512, 640
    layout, codes, scales = random_packed(rows, columns, seed=11)
    plain = PackedEmbedding(layout, dtype=torch.float16)
    fast = PackedEmbedding(layout, dtype=torch.float16, canonical_rows=True)
    load_packed(plain, codes, scales)
    load_packed(fast, codes, scales)
    ids = torch.randint(0, rows, (300,), device="cuda")
    np.testing.assert_array_equal(plain(ids).cpu().numpy(), fast(ids).cpu().numpy())
    assert not hasattr(plain, "_row_blocks")


# -- functional surface ---------------------------------------------------------------------

SINGLE = MatmulConfig(threads=256, batch_tile=1, padded_lut=True, safe_clamp=False, k_split=1)
BATCHED = MatmulConfig(threads=256, batch_tile=4, padded_lut=False, safe_clamp=False, k_split=1)


@pytest.mark.parametrize("config", (SINGLE, BATCHED), ids=("single", "batched"))
def test_tq1_matmul_takes_the_reference_arguments_and_matches_lut23_bit_for_bit(config) -> None:
    rows, columns, batch = 512, 640, 5
    layout, codes, scales = random_packed(rows, columns, seed=3)
    c, s = device_pair(codes, scales)
    x = np.random.default_rng(3).normal(0, 1, size=(batch, columns)).astype(np.float32)
    got = tq1_matmul(c, s, torch.from_numpy(x).cuda(), groups_per_row=layout.groups_per_row, tile=layout.tile,
                     config=config).cpu().numpy()
    want = O.lut23_matmul(blocks_of(layout, codes, scales), x, rows=rows, columns=columns)
    np.testing.assert_array_equal(got, want)


def test_tq1_matmul_split_and_automatic_stay_inside_the_oracle_tolerance() -> None:
    rows, columns = 2048, 5120
    layout, codes, scales = random_packed(rows, columns, seed=4)
    c, s = device_pair(codes, scales)
    x = np.random.default_rng(4).normal(0, 1, size=(1, columns)).astype(np.float32)
    want = O.oracle_matmul(blocks_of(layout, codes, scales), x, rows=rows, columns=columns)
    for config in (MatmulConfig(), MatmulConfig(threads=256, batch_tile=1, padded_lut=False, safe_clamp=False,
                                                k_split=40)):
        got = tq1_matmul(c, s, torch.from_numpy(x).cuda(), groups_per_row=layout.groups_per_row, tile=layout.tile,
                         config=config).cpu().numpy()
        assert O.compare(got, want)["normalised_max_abs_error"] <= ORACLE_RELATIVE_TOLERANCE


@pytest.mark.parametrize("batch", (8, 64, 512))
def test_tq1_gemm_takes_the_reference_arguments(batch: int) -> None:
    rows, columns = 1024, 2048
    layout, codes, scales = random_packed(rows, columns, seed=batch)
    c, s = device_pair(codes, scales)
    x = np.random.default_rng(batch).normal(0, 0.5, size=(batch, columns)).astype(np.float16)
    # a reference GemmConfig, by keyword: its Metal tiling fields are accepted
    config = GemmConfig(batch_block=32, row_block=128, k_block=32, simd_rows=2, simd_columns=2,
                        direct_fragments=True, direct_epilogue=True, threadgroup_table=False, safe_clamp=False)
    got = tq1_gemm(c, s, torch.from_numpy(x).cuda(), groups_per_row=layout.groups_per_row, tile=layout.tile,
                   config=config).float().cpu().numpy()
    want = O.oracle_matmul(blocks_of(layout, codes, scales), x.astype(np.float64), rows=rows, columns=columns)
    # one fp16 rounding of the store (src/ternel_mlx/kernel_gate.py:113: 2e-3)
    assert O.compare(got, want)["normalised_max_abs_error"] <= 2e-3


@pytest.mark.parametrize("dtype", (torch.float32, torch.bfloat16))
def test_tq1_gemm_with_wide_activations_keeps_their_precision(dtype) -> None:
    """bf16 and fp32 prefill run through the LUT23 kernel (fp32 arithmetic), in
    several launches when the batch outgrows one launch's split counters."""
    rows, columns, batch = 4096, 5120, 1100
    layout, codes, scales = random_packed(rows, columns, seed=9)
    c, s = device_pair(codes, scales)
    x = torch.from_numpy(np.random.default_rng(9).normal(0, 1, size=(batch, columns)).astype(np.float32))
    x = x.to(dtype)
    got = tq1_gemm(c, s, x.cuda(), groups_per_row=layout.groups_per_row, tile=layout.tile).float().cpu().numpy()
    sample = np.arange(0, rows, 7)
    blocks = blocks_of(layout, codes, scales)
    want = O.oracle_matmul(blocks[sample], x.float().numpy(), rows=len(sample), columns=columns)
    tol = 1e-5 if dtype == torch.float32 else 1e-2  # src/ternel_mlx/kernel_gate.py:113
    assert O.compare(got[:, sample], want)["normalised_max_abs_error"] <= tol


@pytest.mark.parametrize("index_dtype", (torch.int32, torch.int64, torch.uint32))
def test_tq1_get_rows_takes_the_reference_arguments(index_dtype) -> None:
    rows, columns = 512, 640
    layout, codes, scales = random_packed(rows, columns, seed=6)
    c, s = device_pair(codes, scales)
    ids = np.array([0, 511, 17, 17, 300], dtype=np.int64)
    got = tq1_get_rows(c, s, torch.from_numpy(ids).to(index_dtype).cuda(), groups_per_row=layout.groups_per_row,
                       tile=layout.tile, dtype=torch.float16, threads=256, safe_clamp=False).cpu().numpy()
    want = O.get_rows_reference(blocks_of(layout, codes, scales), ids, rows=rows, columns=columns,
                                dtype=np.float16)
    np.testing.assert_array_equal(got, want)


def test_packed_matmul_takes_codes_and_scales() -> None:
    rows, columns = 256, 384
    layout, codes, scales = random_packed(rows, columns, seed=12)
    module = PackedLinear(layout)
    load_packed(module, codes, scales)
    c, s = device_pair(codes, scales)
    x = torch.randn(3, columns, device="cuda", dtype=torch.float16)
    np.testing.assert_array_equal(packed_matmul(c, s, x, layout=layout).cpu().numpy(), module(x).cpu().numpy())
    np.testing.assert_array_equal(packed_matmul(module.codes, module.scales, x, layout=layout).cpu().numpy(),
                                  module(x).cpu().numpy())


def test_the_functional_cache_follows_in_place_writes() -> None:
    rows, columns = 256, 256
    layout, codes, scales = random_packed(rows, columns, seed=13)
    c, s = device_pair(codes, scales)
    x = torch.randn(1, columns, device="cuda", dtype=torch.float32)
    kw = dict(groups_per_row=layout.groups_per_row, tile=layout.tile, config=SINGLE)
    first = tq1_matmul(c, s, x, **kw)
    assert words_of(c, s, groups_per_row=layout.groups_per_row, tile=layout.tile)[0] is words_of(
        c, s, groups_per_row=layout.groups_per_row, tile=layout.tile)[0]
    c[:, 0, 0, :] = 121  # every row's first five weights become zero
    second = tq1_matmul(c, s, x, **kw).cpu().numpy()
    codes2 = c.cpu().numpy()
    np.testing.assert_array_equal(second, O.lut23_matmul(blocks_of(layout, codes2, scales), x.cpu().numpy(),
                                                         rows=rows, columns=columns))
    assert not np.array_equal(second, first.cpu().numpy())


def test_functional_checks_use_the_reference_messages() -> None:
    layout, codes, scales = random_packed(256, 256, seed=1)
    c, s = device_pair(codes, scales)
    x = torch.zeros(1, 256, device="cuda")
    with pytest.raises(FormatError, match=r"codes shape \(1, 2, 26, 256\) does not match \(tiles, 3, 26, 256\)"):
        tq1_matmul(c, s, x, groups_per_row=3, tile=256)
    with pytest.raises(FormatError, match="codes must be uint8"):
        tq1_matmul(c.to(torch.int32), s, x, groups_per_row=2, tile=256)
    with pytest.raises(FormatError, match="k split 3 does not divide the tensor's 2 groups per row"):
        tq1_matmul(c, s, x, groups_per_row=2, tile=256, config=MatmulConfig(k_split=3))
    with pytest.raises(FormatError, match="activations have 128 columns, expected 256"):
        tq1_matmul(c, s, torch.zeros(1, 128, device="cuda"), groups_per_row=2, tile=256)
    with pytest.raises(FormatError, match="threads must be a positive multiple"):
        MatmulConfig(threads=48)
    with pytest.raises(FormatError, match="out-of-range base-3 bytes: regular=1"):
        bad = c.clone()
        bad[0, 0, 3, 9] = 243
        tq1_matmul(bad, s, x, groups_per_row=2, tile=256)


# -- state --------------------------------------------------------------------------------

def test_state_dict_keys_are_codes_and_scales_of_the_reference_shapes() -> None:
    layout, codes, scales = random_packed(512, 640, seed=21)
    module = PackedLinear(layout)
    load_packed(module, codes, scales)
    state = module.state_dict()
    assert sorted(state) == ["codes", "scales"]
    assert tuple(state["codes"].shape) == layout.codes_shape and state["codes"].dtype == torch.uint8
    assert tuple(state["scales"].shape) == layout.scales_shape and state["scales"].dtype == torch.uint16
    np.testing.assert_array_equal(state["codes"].cpu().numpy(), codes)
    np.testing.assert_array_equal(state["scales"].cpu().numpy(), scales)


def test_load_state_dict_of_artifact_shaped_tensors() -> None:
    model = nn.Sequential(nn.Embedding(512, 256), nn.Linear(256, 384, bias=False))
    from ternel_amd.modules import replace_with_packed

    replace_with_packed(model, embedding_dtype=torch.float32)
    state = {}
    pairs = {}
    for name, rows, columns in (("0", 512, 256), ("1", 384, 256)):
        layout, codes, scales = random_packed(rows, columns, seed=int(name) + 30)
        pairs[name] = (layout, codes, scales)
        state[f"{name}.codes"], state[f"{name}.scales"] = device_pair(codes, scales)
    model.load_state_dict(state, strict=True)
    x = torch.randn(2, 256, device="cuda")
    layout, codes, scales = pairs["1"]
    want = O.oracle_matmul(blocks_of(layout, codes, scales), x.cpu().numpy(), rows=384, columns=256)
    assert O.compare(model[1](x).cpu().numpy(), want)["normalised_max_abs_error"] <= ORACLE_RELATIVE_TOLERANCE
    round_trip = {k: v.cpu() for k, v in model.state_dict().items()}
    for k, v in state.items():
        assert torch.equal(round_trip[k], v.cpu())


def test_a_strict_load_rejects_a_missing_or_mis_shaped_packed_tensor() -> None:
    layout, codes, scales = random_packed(256, 256, seed=2)
    module = PackedLinear(layout)
    c, s = device_pair(codes, scales)
    with pytest.raises(RuntimeError, match="Missing key"):
        module.load_state_dict({"codes": c}, strict=True)
    with pytest.raises(RuntimeError, match="does not match"):
        module.load_state_dict({"codes": c[:, :1].contiguous(), "scales": s}, strict=True)


def test_assigning_codes_or_scales_converts_on_the_gpu() -> None:
    layout, codes, scales = random_packed(256, 256, seed=23)
    _, codes2, scales2 = random_packed(256, 256, seed=24)
    module = PackedLinear(layout)
    load_packed(module, codes, scales)
    c2, s2 = device_pair(codes2, scales2)
    module.codes = c2
    module.scales = s2
    np.testing.assert_array_equal(module.codes.cpu().numpy(), codes2)
    np.testing.assert_array_equal(module.scales.cpu().numpy(), scales2)
    np.testing.assert_array_equal(module.blocks.cpu().numpy(), blocks_of(layout, codes2, scales2))
