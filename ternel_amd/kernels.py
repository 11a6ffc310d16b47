"""Functional entry points over the gfx950 library (mirror of src/ternel_mlx/kernels.py:951-1398).

``tq1_matmul`` (LUT23: decode GEMV and small batches), ``tq1_gemm`` (MFMA:
prefill) and ``tq1_get_rows`` (embedding gather) take the *packed* device
weight -- the canonical 28-byte blocks permuted into 64-row word-interleaved
tiles, a uint32 tensor of shape ``(ceil(rows/64), groups_per_row, 7, 64)`` made
by :func:`pack_weights` -- check every argument on the host and raise
``FormatError`` before anything is launched, as the reference's wrappers do
(``_check_packed``/``_check_activations``, kernels.py:1191-1212, 1274-1284).
Outputs are fresh tensors in the activation dtype.

Split-K workspaces: the LUT23 kernel reduces its K chunks inside the launch
through arrival counters that must start at zero and are left at zero, so the
workspace is allocated zero-filled once per device and reused.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .format import BLOCK_BYTES, FormatError, as_device_blocks
from .layout import PackedTensorLayout

ACTIVATION_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_DTYPE_CODE = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}

TILE_ROWS = 64
BLOCK_WORDS = 7
LUT23_THREADS = 256
LUT23_BATCH_TILES = (1, 2, 4)


@dataclass(frozen=True)
class MatmulConfig:
    """LUT23 knobs (src/ternel_mlx/kernels.py:963-1006): batch tile and K split.

    ``0`` means automatic: a batch tile of 1 (fastest at every measured 27B
    shape) and the split measured best for the shape's groups per row.
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


GEMM_FORMS = {"auto": 0, "tile": 1, "direct": 2, "wide": 3}
DIRECT_MAX_BATCH = 64


@dataclass(frozen=True)
class GemmConfig:
    """MFMA knobs: the kernel form and the K split (0 = automatic).

    ``form`` picks how weight fragments reach the matrix cores, like the
    reference's ``direct_fragments`` switch (src/ternel_mlx/kernels.py:1043-1188):
    ``"tile"`` decodes 128x128 weight tiles into LDS (prefill), ``"direct"``
    decodes straight into MFMA operand registers (at most 64 activation rows),
    ``"wide"`` decodes into the operand registers of 256-row output tiles (32
    to 256 activation rows wide) split stream-K over the CUs (prefill; K split
    0 or 1), ``"auto"`` takes ``"direct"`` up to 32 rows and, above, ``"wide"``
    when it has enough tiles (CUs/4) or work per CU (15 steps) for its stream-K
    reduction to pay, ``"tile"`` otherwise (and whenever a K split above 1 is
    fixed).
    """

    k_split: int = 0
    form: str = "auto"

    def __post_init__(self) -> None:
        if self.k_split < 0:
            raise FormatError(f"k split must be positive, got {self.k_split}")
        if self.form not in GEMM_FORMS:
            raise FormatError(f"GEMM form must be one of {sorted(GEMM_FORMS)}, got {self.form!r}")

    @property
    def benchmark_name(self) -> str:
        name = "gemm_128x128" if self.form == "tile" else f"gemm_{self.form}"
        return name if self.k_split in (0, 1) else f"{name}_k{self.k_split}"


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def packed_shape(layout: PackedTensorLayout) -> tuple[int, int, int, int]:
    return (math.ceil(layout.rows / TILE_ROWS), layout.groups_per_row, BLOCK_WORDS, TILE_ROWS)


def pack_weights(blocks, *, layout: PackedTensorLayout) -> torch.Tensor:
    """Canonical blocks (host or device) -> packed device words (exact permutation)."""
    device_blocks = as_device_blocks(blocks)
    if device_blocks.shape[0] != layout.groups:
        raise FormatError(
            f"expected {layout.groups} blocks for {layout.rows}x{layout.columns}, got {device_blocks.shape[0]}"
        )
    packed = torch.empty(packed_shape(layout), dtype=torch.int32, device=device_blocks.device)
    assert packed.numel() == _lib.lib().ternel_tq1_packed_words(layout.rows, layout.columns)
    _lib.check(_lib.lib().ternel_tq1_interleave(device_blocks.data_ptr(), layout.rows, layout.columns,
                                                packed.data_ptr(), _stream(device_blocks.device)))
    return packed


def unpack_weights(packed: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """Packed device words -> canonical ``(rows, G, 28)`` uint8 device blocks."""
    check_packed(packed, layout=layout)
    blocks = torch.empty(layout.canonical_shape, dtype=torch.uint8, device=packed.device)
    _lib.check(_lib.lib().ternel_tq1_deinterleave(packed.data_ptr(), layout.rows, layout.columns,
                                                  blocks.data_ptr(), _stream(packed.device)))
    return blocks


def check_packed(packed: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    if not isinstance(packed, torch.Tensor):
        raise FormatError("packed weights must be a torch tensor on the GPU")
    if packed.dtype not in (torch.int32, torch.uint32):
        raise FormatError(f"packed weights must be 32-bit words, got {packed.dtype}")
    if tuple(packed.shape) != packed_shape(layout):
        raise FormatError(f"packed weights of shape {tuple(packed.shape)} do not match {packed_shape(layout)}")
    if not packed.is_cuda:
        raise FormatError("packed weights must live on the GPU")
    if not packed.is_contiguous():
        raise FormatError("packed weights must be contiguous")
    return packed


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


_WORKSPACES: dict[int, torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Zero-initialised split-K scratch, one per device, grown on demand.

    The LUT23 kernel leaves its arrival counters at zero after every launch, so
    the buffer only needs zeroing when it is created -- which never happens
    inside a graph capture once an eager call of the same size has run. Calls
    sharing the buffer must not run concurrently (one stream per device).
    """
    if nbytes == 0:
        return None
    key = device.index if device.index is not None else torch.cuda.current_device()
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("split-K workspace must be sized by an eager call before graph capture")
        buf = torch.zeros(max(nbytes, 1 << 22), dtype=torch.uint8, device=device)
        torch.cuda.synchronize(device)
        _WORKSPACES[key] = buf
    return buf


def tq1_matmul(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout,
               config: MatmulConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` through the LUT23 kernel; ``(batch, rows)`` in ``x.dtype``.

    Reference: tq1_matmul, src/ternel_mlx/kernels.py:1215-1271. A ``k_split`` that
    does not divide the group count is refused, as there.
    """
    config = config or MatmulConfig()
    check_packed(packed, layout=layout)
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
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_matmul(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns,
        _DTYPE_CODE[x.dtype], config.batch_tile, config.k_split,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(x.device)))
    return out


def tq1_gemm(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout,
             config: GemmConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` on the MFMA kernel (fp16 activations); reference tq1_gemm, kernels.py:1287-1357."""
    config = config or GemmConfig()
    check_packed(packed, layout=layout)
    batch = check_activations(x, layout=layout)
    if x.dtype != torch.float16:
        raise FormatError(f"the MFMA path takes float16 activations, got {x.dtype}")
    if config.k_split and layout.groups_per_row % config.k_split:
        raise FormatError(
            f"k split {config.k_split} does not divide the tensor's {layout.groups_per_row} groups per row"
        )
    if config.form == "direct" and batch > DIRECT_MAX_BATCH:
        raise FormatError(f"the direct-fragment form takes at most {DIRECT_MAX_BATCH} activation rows, got {batch}")
    form = GEMM_FORMS[config.form]
    x = x.contiguous()
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    need = handle.ternel_tq1_gemm_workspace_bytes(batch, layout.rows, layout.columns, form, config.k_split)
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_gemm(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns,
        _lib.DTYPE_F16, form, config.k_split, ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _stream(x.device)))
    return out


def tq1_linear(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """The library's own dispatch (``ternel_tq1_linear``) for a 2-D ``x``."""
    check_packed(packed, layout=layout)
    batch = check_activations(x, layout=layout)
    x = x.contiguous()
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    code = _DTYPE_CODE[x.dtype]
    need = handle.ternel_tq1_linear_workspace_bytes(batch, layout.rows, layout.columns, code)
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_linear(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns, code,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(x.device)))
    return out


def tq1_swiglu(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """SiLU(gate) * up of a SwiGLU MLP whose gate and up projections are one
    packed weight with alternating rows (``layout.interleave_gate_up``):
    ``(batch, rows // 2)`` in ``x.dtype``, each gate/up value rounded to
    ``x.dtype`` as the unfused layers would return it."""
    check_packed(packed, layout=layout)
    batch = check_activations(x, layout=layout)
    if layout.rows % 2:
        raise FormatError(f"a SwiGLU weight interleaves gate and up rows, so its rows must be even, "
                          f"got {layout.rows}")
    x = x.contiguous()
    out = torch.empty((batch, layout.rows // 2), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    code = _DTYPE_CODE[x.dtype]
    need = handle.ternel_tq1_swiglu_workspace_bytes(batch, layout.rows, layout.columns, code)
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_swiglu(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns, code,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(x.device)))
    return out


def _gather_ids(indices: torch.Tensor, dtype: torch.dtype, device) -> torch.Tensor:
    if dtype not in ACTIVATION_DTYPES:
        raise FormatError(f"output dtype must be one of {ACTIVATION_DTYPES}, got {dtype}")
    if indices.ndim != 1:
        raise FormatError(f"indices must be 1-D, got shape {tuple(indices.shape)}")
    if indices.numel() <= 0:
        raise FormatError("indices are empty")
    if indices.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8):
        raise FormatError(f"indices must be an integer tensor, got {indices.dtype}")
    return indices.to(device=device, dtype=torch.int64).contiguous()


def tq1_get_rows(packed: torch.Tensor, indices: torch.Tensor, *, layout: PackedTensorLayout,
                 dtype: torch.dtype) -> torch.Tensor:
    """Decode the rows named by ``indices`` (1-D); reference tq1_get_rows, kernels.py:1360-1398.

    Ids outside ``[0, rows)`` read as zeros, as the reference kernel does.
    """
    check_packed(packed, layout=layout)
    ids = _gather_ids(indices, dtype, packed.device)
    out = torch.empty((ids.numel(), layout.columns), dtype=dtype, device=packed.device)
    _lib.check(_lib.lib().ternel_tq1_get_rows(
        packed.data_ptr(), layout.rows, layout.columns, ids.data_ptr(), ids.numel(), out.data_ptr(),
        _DTYPE_CODE[dtype], _stream(packed.device)))
    return out


def tq1_get_rows_canonical(blocks: torch.Tensor, indices: torch.Tensor, *, layout: PackedTensorLayout,
                           dtype: torch.dtype) -> torch.Tensor:
    """``tq1_get_rows`` over canonical ``(rows, G, 28)`` uint8 device blocks (``unpack_weights``):
    a token's blocks are one contiguous run, so a gather reads only the rows it returns."""
    if blocks.dtype != torch.uint8 or tuple(blocks.shape) != tuple(layout.canonical_shape):
        raise FormatError(f"canonical blocks must be uint8 {tuple(layout.canonical_shape)}, "
                          f"got {blocks.dtype} {tuple(blocks.shape)}")
    if blocks.device.type != "cuda" or not blocks.is_contiguous():
        raise FormatError("canonical blocks must be a contiguous device tensor")
    ids = _gather_ids(indices, dtype, blocks.device)
    out = torch.empty((ids.numel(), layout.columns), dtype=dtype, device=blocks.device)
    _lib.check(_lib.lib().ternel_tq1_get_rows_canonical(
        blocks.data_ptr(), layout.rows, layout.columns, ids.data_ptr(), ids.numel(), out.data_ptr(),
        _DTYPE_CODE[dtype], _stream(blocks.device)))
    return out


__all__ = [
    "ACTIVATION_DTYPES",
    "BLOCK_BYTES",
    "GemmConfig",
    "MatmulConfig",
    "pack_weights",
    "packed_shape",
    "tq1_gemm",
    "tq1_get_rows",
    "tq1_get_rows_canonical",
    "tq1_linear",
    "tq1_matmul",
    "unpack_weights",
]
