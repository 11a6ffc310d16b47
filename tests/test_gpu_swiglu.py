"""Fused SwiGLU (gate and up as one packed weight, SiLU(gate) * up in the
epilogue) against the unfused layers and the fp64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, random_blocks, to_dev
from ternel_amd.format import FormatError
from ternel_amd.kernels import tq1_swiglu_words
from ternel_amd.layout import interleave_gate_up
from ternel_amd.modules import PackedLinear, PackedSwiGLU

pytestmark = pytest.mark.gpu

NORTH_STAR_TOLERANCE = 1e-3


def unfused(gate_blocks, up_blocks, x: torch.Tensor, *, with_operands: bool = False):
    """The two packed linears, then SiLU(g) * u in fp32 from their rounded outputs."""
    hidden, g, _ = gate_blocks.shape
    gate, up = PackedLinear(layout(hidden, g * 128)), PackedLinear(layout(hidden, g * 128))
    gate.load_blocks(gate_blocks)
    up.load_blocks(up_blocks)
    gv, uv = gate(x).float(), up(x).float()
    z = (gv / (1.0 + torch.exp(-gv)) * uv).to(x.dtype)
    return (z, gv, uv) if with_operands else z


def fp16_spacing(v: torch.Tensor) -> torch.Tensor:
    """Distance from |v| to the next fp16 value (2**-24 below the normal range)."""
    exponent = torch.frexp(v).exponent
    return torch.ldexp(torch.ones_like(v), exponent - 11).clamp_min(2.0 ** -24)


def spacing(v: torch.Tensor, dtype) -> torch.Tensor:
    """Distance from |v| to the next value of ``dtype`` (fp16, bf16 or fp32)."""
    if dtype == torch.float16:
        return fp16_spacing(v)
    bits = {torch.bfloat16: 8, torch.float32: 24}[dtype]
    return torch.ldexp(torch.ones_like(v), torch.frexp(v).exponent - bits).clamp_min(2.0 ** -126)


def oracle(gate_blocks, up_blocks, x: np.ndarray) -> np.ndarray:
    hidden, g, _ = gate_blocks.shape
    gv = O.oracle_matmul(gate_blocks, x, rows=hidden, columns=g * 128)
    uv = O.oracle_matmul(up_blocks, x, rows=hidden, columns=g * 128)
    return gv / (1.0 + np.exp(-gv)) * uv


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
@pytest.mark.parametrize("batch", (1, 3, 4, 16, 70))
@pytest.mark.parametrize(("hidden", "columns"), ((512, 1024), (300, 640), (2048, 5120)))
def test_fused_swiglu_matches_the_unfused_layers(dtype, batch: int, hidden: int, columns: int) -> None:
    gate_blocks = random_blocks(hidden, columns, seed=hidden + batch)
    up_blocks = random_blocks(hidden, columns, seed=hidden + batch + 1)
    x_np = np.random.default_rng(batch + hidden).normal(0, 1, size=(batch, columns)).astype(np.float32)
    x = to_dev(x_np).to(dtype)
    mlp = PackedSwiGLU(hidden, columns)
    mlp.load_blocks(gate_blocks, up_blocks)
    got = mlp(x)
    assert got.dtype == dtype and got.shape == (batch, hidden)
    want, gv, uv = unfused(gate_blocks, up_blocks, x, with_operands=True)
    diff = (got.float() - want.float()).abs()
    if (dtype != torch.float32 and batch > 4) or batch == 1:
        # The GEMM path (fp16, and bf16 on the wide form), and at one vector the LUT kernel's automatic
        # K split (chosen from the row count), cut a 2 x hidden weight
        # differently from a hidden one, so the fp32 sums
        # differ by up to the accumulation bound (columns x eps x |x||W|, per
        # operand) and may then round to another value of the activation type
        # (a step of either neighbouring binade); z moves by at most that
        # through its partial derivatives, plus one step of its own rounding.
        xa = np.abs(x.float().cpu().numpy().astype(np.float64))
        eps = float(np.finfo(np.float32).eps)
        accumulation = [torch.from_numpy(columns * eps * (xa @ np.abs(O.dense_weights(b, rows=hidden,
                                                                                      columns=columns)).T)).cuda()
                        for b in (gate_blocks, up_blocks)]
        dg = 2 * accumulation[0] + 2 * spacing(gv, dtype)
        du = 2 * accumulation[1] + 2 * spacing(uv, dtype)
        sig = torch.sigmoid(gv)
        dz_dg = (uv * sig * (1.0 + gv * (1.0 - sig))).abs()
        dz_du = (gv * sig).abs()
        bound = 1.01 * (dz_dg * dg + dz_du * du) + spacing(want.float(), dtype)
        assert bool((diff <= bound).all()), float((diff - bound).max())
    else:
        # The LUT path (batches of 2 to 4 here, every fp32 batch) sums each row
        # in the same chunk order for the fused and the separate weights: gate
        # and up round to the same values and z agrees to SiLU's exp (an fp32
        # ulp against torch's) and one rounding step of z.
        ulp = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7, torch.float32: 2.0 ** -22}[dtype]
        assert bool((diff <= ulp * want.float().abs() + 1e-30).all()), float(diff.max())
    ref = oracle(gate_blocks, up_blocks, x.float().cpu().numpy().astype(np.float64))
    result = O.compare(got.float().cpu().numpy(), ref)
    # z combines two values each rounded once to the activation type (as the
    # unfused layers return them), so its error is up to about twice a single
    # projection's: the north star's 1e-3 for each operand.
    bound = {torch.float16: 2 * NORTH_STAR_TOLERANCE + 2.0 ** -11, torch.bfloat16: 2e-2,
             torch.float32: 1e-5}[dtype]
    assert result["normalised_max_abs_error"] < bound
    assert result["pattern_mismatches"] == 0


def test_the_fused_weight_is_the_interleaved_gate_and_up() -> None:
    gate_blocks, up_blocks = random_blocks(256, 512, seed=1), random_blocks(256, 512, seed=2)
    mlp = PackedSwiGLU(256, 512)
    mlp.load_blocks(gate_blocks, up_blocks)
    assert torch.equal(mlp.packed, pack(interleave_gate_up(gate_blocks, up_blocks)))
    x = torch.randn(2, 5, 512, device="cuda", dtype=torch.float16)
    assert mlp(x).shape == (2, 5, 256)


def test_an_odd_row_count_is_rejected() -> None:
    blocks = random_blocks(255, 256, seed=3)
    with pytest.raises(FormatError, match="rows must be even"):
        tq1_swiglu_words(pack(blocks), torch.zeros((1, 256), device="cuda", dtype=torch.float16), layout=layout(255, 256))


def test_non_finite_gate_values_follow_ieee() -> None:
    hidden, columns = 256, 256
    gate_blocks, up_blocks = random_blocks(hidden, columns, seed=8), random_blocks(hidden, columns, seed=9)
    x = torch.zeros((1, columns), device="cuda", dtype=torch.float32)
    x[0, 7] = float("inf")
    mlp = PackedSwiGLU(hidden, columns)
    mlp.load_blocks(gate_blocks, up_blocks)
    got = mlp(x).cpu().numpy()
    want = unfused(gate_blocks, up_blocks, x).cpu().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[np.isinf(want)], want[np.isinf(want)])
