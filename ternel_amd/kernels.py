"""Functional entry points over the gfx950 library (mirror of src/ternel_mlx/kernels.py:951-1398).

``tq1_matmul`` (LUT23, decode GEMV and small batches), ``tq1_gemm`` (MFMA,
prefill) and ``tq1_get_rows`` (embedding gather) take canonical device blocks
``(rows, groups_per_row, 28)`` uint8, check every argument on the host and raise
``FormatError`` *before* anything is launched, exactly as the reference's
wrappers do (``_check_packed``/``_check_activations``, kernels.py:1191-1212,
1274-1284). Outputs are fresh tensors in the activation dtype; split-K
workspaces are allocated here by torch and handed to the C ABI.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .format import BLOCK_BYTES, BLOCK_SIZE, FormatError
from .layout import PackedTensorLayout

ACTIVATION_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_DTYPE_CODE = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}

# One thread per output row in a 256-lane workgroup (4 wave64s).
LUT23_THREADS = 256
LUT23_BATCH_TILES = (1, 2, 4)


@dataclass(frozen=True)
class MatmulConfig:
    """LUT23 knobs (src/ternel_mlx/kernels.py:963-1006): batch tile and K split.

    ``k_split=0`` lets the library pick the largest divisor of the group count
    that keeps the grid near its MI355X workgroup target.
    """

    batch_tile: int = 0
    k_split: int = 0

    def __post_init__(self) -> None:
        if self.batch_tile not in (0, *LUT23_BATCH_TILES):
            raise FormatError(f"batch tile must be one of {LUT23_BATCH_TILES}, got {self.batch_tile}")
        if self.k_split < 0:
            raise FormatError(f"k split must be positive, got {self.k_split}")

    @property
    def benchmark_name(self) -> str:
        name = f"lut23_bt{self.batch_tile or 'auto'}"
        return name if self.k_split in (0, 1) else f"{name}_k{self.k_split}"


@dataclass(frozen=True)
class GemmConfig:
    """MFMA prefill knobs: the K split (0 = automatic)."""

    k_split: int = 0

    def __post_init__(self) -> None:
        if self.k_split < 0:
            raise FormatError(f"k split must be positive, got {self.k_split}")

    @property
    def benchmark_name(self) -> str:
        return "gemm_128x128" if self.k_split in (0, 1) else f"gemm_128x128_k{self.k_split}"


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def check_blocks(blocks: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """Device canonical blocks of ``layout``'s shape, or FormatError."""
    if not isinstance(blocks, torch.Tensor):
        raise FormatError("blocks must be a torch tensor on the GPU")
    if blocks.dtype != torch.uint8:
        raise FormatError(f"blocks must be uint8, got {blocks.dtype}")
    expected = layout.canonical_shape
    if tuple(blocks.shape) != expected and not (blocks.ndim == 2 and tuple(blocks.shape) == (layout.groups, BLOCK_BYTES)):
        raise FormatError(f"blocks shape {tuple(blocks.shape)} does not match {expected}")
    if not blocks.is_cuda:
        raise FormatError("blocks must live on the GPU")
    if not blocks.is_contiguous():
        raise FormatError("blocks must be contiguous")
    if blocks.data_ptr() % 4:
        raise FormatError("blocks must be 4-byte aligned")
    return blocks


def check_activations(x: torch.Tensor, *, layout: PackedTensorLayout) -> int:
    """src/ternel_mlx/kernels.py:1274-1284, same messages."""
    if x.dtype not in ACTIVATION_DTYPES:
        raise FormatError(f"activations must be one of {ACTIVATION_DTYPES}, got {x.dtype}")
    if x.ndim != 2:
        raise FormatError(f"activations must be 2-D (batch, columns), got shape {tuple(x.shape)}")
    if x.shape[1] != layout.columns:
        raise FormatError(f"activations have {x.shape[1]} columns, expected {layout.columns}")
    if x.shape[0] <= 0:
        raise FormatError("activations have an empty batch dimension")
    if not x.is_cuda:
        raise FormatError("activations must live on the GPU")
    return x.shape[0]


def tq1_matmul(blocks: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout,
               config: MatmulConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` through the LUT23 kernel; ``(batch, rows)`` in ``x.dtype``.

    Reference: tq1_matmul, src/ternel_mlx/kernels.py:1215-1271. A ``k_split`` that
    does not divide the group count is refused, as there.
    """
    config = config or MatmulConfig()
    check_blocks(blocks, layout=layout)
    batch = check_activations(x, layout=layout)
    if config.k_split and layout.groups_per_row % config.k_split:
        raise FormatError(
            f"k split {config.k_split} does not divide the tensor's {layout.groups_per_row} groups per row"
        )
    x = x.contiguous()
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    need = handle.ternel_tq1_matmul_workspace_bytes(batch, layout.rows, layout.columns,
                                                     config.batch_tile, config.k_split)
    ws = torch.empty(max(need, 4), dtype=torch.uint8, device=x.device) if need else None
    _lib.check(handle.ternel_tq1_matmul(
        blocks.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns,
        _DTYPE_CODE[x.dtype], config.batch_tile, config.k_split,
        ws.data_ptr() if ws is not None else None, need, _stream(x.device)))
    return out


def tq1_gemm(blocks: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout,
             config: GemmConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` on the MFMA kernel (fp16 activations); reference tq1_gemm, kernels.py:1287-1357."""
    config = config or GemmConfig()
    check_blocks(blocks, layout=layout)
    batch = check_activations(x, layout=layout)
    if x.dtype != torch.float16:
        raise FormatError(f"the MFMA path takes float16 activations, got {x.dtype}")
    if config.k_split and layout.groups_per_row % config.k_split:
        raise FormatError(
            f"k split {config.k_split} does not divide the tensor's {layout.groups_per_row} groups per row"
        )
    x = x.contiguous()
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    need = handle.ternel_tq1_gemm_workspace_bytes(batch, layout.rows, layout.columns, config.k_split)
    ws = torch.empty(max(need, 4), dtype=torch.uint8, device=x.device) if need else None
    _lib.check(handle.ternel_tq1_gemm(
        blocks.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns,
        _lib.DTYPE_F16, config.k_split, ws.data_ptr() if ws is not None else None, need,
        _stream(x.device)))
    return out


def tq1_linear(blocks: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """The library's own dispatch (``ternel_tq1_linear``) for a 2-D ``x``."""
    check_blocks(blocks, layout=layout)
    batch = check_activations(x, layout=layout)
    x = x.contiguous()
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    code = _DTYPE_CODE[x.dtype]
    need = handle.ternel_tq1_linear_workspace_bytes(batch, layout.rows, layout.columns, code)
    ws = torch.empty(max(need, 4), dtype=torch.uint8, device=x.device) if need else None
    _lib.check(handle.ternel_tq1_linear(
        blocks.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns, code,
        ws.data_ptr() if ws is not None else None, need, _stream(x.device)))
    return out


def tq1_get_rows(blocks: torch.Tensor, indices: torch.Tensor, *, layout: PackedTensorLayout,
                 dtype: torch.dtype) -> torch.Tensor:
    """Decode the rows named by ``indices`` (1-D); reference tq1_get_rows, kernels.py:1360-1398.

    Ids outside ``[0, rows)`` read as zeros, as the reference kernel does.
    """
    check_blocks(blocks, layout=layout)
    if dtype not in ACTIVATION_DTYPES:
        raise FormatError(f"output dtype must be one of {ACTIVATION_DTYPES}, got {dtype}")
    if indices.ndim != 1:
        raise FormatError(f"indices must be 1-D, got shape {tuple(indices.shape)}")
    if indices.numel() <= 0:
        raise FormatError("indices are empty")
    if indices.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8):
        raise FormatError(f"indices must be an integer tensor, got {indices.dtype}")
    ids = indices.to(device=blocks.device, dtype=torch.int64).contiguous()
    out = torch.empty((ids.numel(), layout.columns), dtype=dtype, device=blocks.device)
    _lib.check(_lib.lib().ternel_tq1_get_rows(
        blocks.data_ptr(), layout.rows, layout.columns, ids.data_ptr(), ids.numel(), out.data_ptr(),
        _DTYPE_CODE[dtype], _stream(blocks.device)))
    return out


def lut23_grid(layout: PackedTensorLayout, batch: int, config: MatmulConfig) -> tuple[int, int, int]:
    """Workgroups of a LUT23 launch: (row tiles, batch tiles, K split)."""
    bt = config.batch_tile or (4 if batch >= 4 else 2 if batch >= 2 else 1)
    return (math.ceil(layout.rows / LUT23_THREADS), math.ceil(batch / bt), max(config.k_split, 1))
