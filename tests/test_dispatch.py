"""The dispatch rule replayed against a measured MI355X sweep, as the reference
replays its Metal sweeps through select_gemm (tests/test_mlx_modules.py:553,
1007). tests/golden/dispatch_sweep_mi355x.json holds the time of every kernel
the library can run for each (27B linear shape, batch), measured by
tests/golden/sweep_dispatch.py; the rule must pick one within 15 % of the
fastest everywhere."""

from __future__ import annotations

import json

import pytest
import torch

from tests.conftest import GOLDEN
from ternel_amd import _lib
from ternel_amd.layout import PackedTensorLayout
from ternel_amd.modules import select_kernel

SWEEP = json.loads((GOLDEN / "dispatch_sweep_mi355x.json").read_text())
NAMES = {100: "lut23", 1: "tile", 2: "direct", 3: "wide"}


@pytest.mark.parametrize("row", SWEEP["rows"], ids=lambda r: f"{r['shape']}-M{r['M']}")
def test_the_rule_picks_a_kernel_within_15_percent_of_the_fastest(row) -> None:
    code = _lib.lib().ternel_tq1_linear_kernel(row["M"], row["N"], row["K"], _lib.DTYPE_F16)
    chosen = NAMES[code]
    times = row["us"]
    assert chosen in times, f"the rule picked {chosen}, which the sweep did not time"
    assert times[chosen] <= 1.15 * min(times.values()), (chosen, times)


def test_the_module_dispatch_follows_the_library() -> None:
    for row in SWEEP["rows"]:
        layout = PackedTensorLayout.for_tensor(row["N"], row["K"])
        code = _lib.lib().ternel_tq1_linear_kernel(row["M"], row["N"], row["K"], _lib.DTYPE_F16)
        assert select_kernel(layout, row["M"], torch.float16) == ("lut23" if code == 100 else "gemm")


def test_fp32_activations_take_the_lut_kernel_and_bf16_the_wide_form() -> None:
    handle = _lib.lib()
    for M in (1, 3, 8, 64, 512, 2048):
        assert handle.ternel_tq1_linear_kernel(M, 17408, 5120, _lib.DTYPE_F32) == 100
        # bf16: the LUT23 kernel where fp16 takes it, the wide form (3) above
        fp16 = handle.ternel_tq1_linear_kernel(M, 17408, 5120, _lib.DTYPE_F16)
        assert handle.ternel_tq1_linear_kernel(M, 17408, 5120, _lib.DTYPE_BF16) == (100 if fp16 == 100 else 3)


def test_the_sweep_covers_every_regime() -> None:
    chosen = {NAMES[_lib.lib().ternel_tq1_linear_kernel(r["M"], r["N"], r["K"], _lib.DTYPE_F16)] for r in SWEEP["rows"]}
    assert chosen == {"lut23", "direct", "wide", "tile"}
