"""ternel_tq1_matmul_noalloc (the workspace-free LUT23 product) against
ternel_tq1_matmul with a caller workspace, through the C ABI: two calls in a
row, the second smaller, bit-identical outputs (same kernels, same split,
same summation order), and the host-side rejection of a split too large for
the static scratch."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import tq1_oracle as O
from ternel_amd import _lib, synthetic
from ternel_amd.format import FormatError
from ternel_amd.kernels import pack_weights
from ternel_amd.layout import PackedTensorLayout

pytestmark = pytest.mark.gpu

DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def with_workspace(packed, x, rows: int, columns: int, batch_tile: int, k_split: int) -> torch.Tensor:
    M = x.shape[0]
    y = torch.empty((M, rows), dtype=x.dtype, device="cuda")
    need = _lib.lib().ternel_tq1_matmul_workspace_bytes(M, rows, columns, batch_tile, k_split)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    _lib.check(_lib.lib().ternel_tq1_matmul(packed.data_ptr(), x.data_ptr(), y.data_ptr(), M, rows, columns,
                                            DTYPES[x.dtype], batch_tile, k_split, ws.data_ptr(), need,
                                            torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return y


def without_workspace(packed, x, rows: int, columns: int, batch_tile: int, k_split: int) -> torch.Tensor:
    M = x.shape[0]
    y = torch.empty((M, rows), dtype=x.dtype, device="cuda")
    _lib.check(_lib.lib().ternel_tq1_matmul_noalloc(packed.data_ptr(), x.data_ptr(), y.data_ptr(), M, rows,
                                                    columns, DTYPES[x.dtype], batch_tile, k_split,
                                                    torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return y


def weight(rows: int, columns: int, seed: int):
    lay = PackedTensorLayout.for_tensor(rows, columns)
    blocks = synthetic.device_blocks(rows, columns, seed=seed)
    return blocks, pack_weights(blocks, layout=lay)


# (rows, columns, M, dtype, batch_tile, k_split): the first call of each pair
# is the larger. 64 gate/up vectors need 44.6 MB of partials, so the
# workspace-free call runs them as three launches of at most 24 vectors, where
# the workspace call runs two (its counter region holds 60).
CALL_PAIRS = (
    ((17408, 5120, 64, torch.float16, 0, 0), (4096, 4096, 1, torch.float16, 0, 0)),
    ((5120, 17408, 6, torch.bfloat16, 2, 0), (5120, 8192, 2, torch.bfloat16, 1, 8)),
    ((8192, 5120, 4, torch.float32, 4, 10), (640, 1024, 3, torch.float32, 1, 2)),
    # one vector over 136 and then 64 groups: the strip GEMV in four, then
    # two, K chunks, met in the scratch's counter region
    ((5120, 17408, 1, torch.float16, 0, 0), (5120, 8192, 1, torch.float16, 0, 0)),
)


@pytest.mark.parametrize("pair", CALL_PAIRS, ids=lambda p: "-".join(str(v) for v in p[0][:3]))
def test_two_calls_match_the_workspace_entry_point(pair) -> None:
    for n, (rows, columns, M, dtype, batch_tile, k_split) in enumerate(pair):
        print(f"call {n}: rows={rows} columns={columns} M={M} {dtype} batch_tile={batch_tile} k_split={k_split}",
              flush=True)
        blocks, packed = weight(rows, columns, seed=synthetic.SEED_BASE + 70 + n)
        x = synthetic.device_activations(M, columns, seed=synthetic.SEED_BASE + 71 + n).to(dtype)
        got = without_workspace(packed, x, rows, columns, batch_tile, k_split)
        want = with_workspace(packed, x, rows, columns, batch_tile, k_split)
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), \
            float((got.float() - want.float()).abs().max())
        # and the shared product against the fp64 oracle on sampled rows
        sample = np.sort(np.random.default_rng(rows + M).choice(rows, size=64, replace=False))
        oracle = O.oracle_matmul(blocks[torch.from_numpy(sample).cuda()].cpu().numpy(),
                                 x.float().cpu().numpy().astype(np.float64), rows=len(sample), columns=columns)
        tolerance = {torch.float16: 1e-3, torch.bfloat16: 1e-2, torch.float32: 1e-5}[dtype]
        assert O.compare(got.float().cpu().numpy()[:, sample], oracle)["normalised_max_abs_error"] < tolerance


def test_a_split_too_large_for_the_scratch_is_rejected_or_dropped() -> None:
    # 450048 rows x 5120 columns: a requested split of 40 needs 72 MB of
    # partials for one vector, the automatic split of 10 needs 18 MB; both
    # are over the scratch's 16 MiB.
    rows, columns = 450048, 40 * 128
    rc = _lib.lib().ternel_tq1_matmul_noalloc(None, None, None, 1, rows, columns, _lib.DTYPE_F16, 1, 40,
                                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.TERNEL_TQ1_EINVAL
    assert "more than the 16777216 bytes of the static scratch" in _lib.last_error()
    with pytest.raises(FormatError, match="static scratch"):
        _lib.check(rc)
    # the automatic split runs unsplit: the same sums as a requested split of one
    print(f"unsplit call: rows={rows} columns={columns}", flush=True)
    blocks, packed = weight(rows, columns, seed=3)
    x = synthetic.device_activations(1, columns, seed=4)
    got = without_workspace(packed, x, rows, columns, 0, 0)
    want = with_workspace(packed, x, rows, columns, 1, 1)
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))
    sample = np.sort(np.random.default_rng(9).choice(rows, size=64, replace=False))
    oracle = O.oracle_matmul(blocks[torch.from_numpy(sample).cuda()].cpu().numpy(),
                             x.float().cpu().numpy().astype(np.float64), rows=len(sample), columns=columns)
    assert O.compare(got.float().cpu().numpy()[:, sample], oracle)["normalised_max_abs_error"] < 1e-3
