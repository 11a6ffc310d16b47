"""Functional entry points over the gfx950 library (mirror of src/ternel_mlx/kernels.py:951-1398).

Two surfaces over the same kernels:

* the reference's own signatures -- ``tq1_matmul(codes, scales, x, *,
  groups_per_row, tile, config)``, ``tq1_gemm(...)`` and ``tq1_get_rows(codes,
  scales, indices, *, groups_per_row, tile, dtype, threads, safe_clamp)`` --
  over the reference's tiled pair (``codes`` uint8 ``(tiles, G, 26, tile)``,
  ``scales`` uint16 raw fp16 bits ``(tiles, G, tile)``) as device tensors. The
  pair is converted once, on the GPU, into the engine's packed words and the
  result cached for as long as both tensors live unchanged (their storage and
  version counters key the cache), so repeated calls pay nothing for it;
* the engine's own ``*_words`` functions over packed words (``pack_weights``),
  which the modules use.

Every argument is checked on the host and ``FormatError`` raised before
anything is launched, with the reference's messages (``_check_packed`` /
``_check_activations``, kernels.py:1191-1212, 1274-1284). Outputs are fresh
tensors in the activation dtype.

Split-K workspaces: kernels that reduce K chunks inside the launch use arrival
counters and piece slots that start at zero and are left at zero, so each
(device, stream) gets one zero-filled workspace, reused.
"""

from __future__ import annotations

import ctypes
import math
import weakref
from collections import OrderedDict
from dataclasses import dataclass

import torch

from . import _lib
from .format import BLOCK_BYTES, BLOCK_SIZE, CODE_SLOTS, FormatError, as_device_blocks
from .layout import PackedTensorLayout

ACTIVATION_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_DTYPE_CODE = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}

TILE_ROWS = 64
BLOCK_WORDS = 7
LUT23_THREADS = 256
LUT23_BATCH_TILES = (1, 2, 4)


@dataclass(frozen=True)
class MatmulConfig:
    """LUT23 knobs, with the reference's fields (src/ternel_mlx/kernels.py:963-1006).

    ``batch_tile`` (1, 2 or 4 vectors per workgroup) and ``k_split`` (K chunks,
    dividing the groups per row, reduced in chunk order) are honoured; ``0``
    means automatic for both -- one vector per workgroup and the split measured
    best for the shape. ``threads``,
    ``padded_lut`` and ``safe_clamp`` are the Metal kernel's own template knobs:
    they are validated as the reference validates them and otherwise have no
    effect (the gfx950 kernels fix their workgroup sizes, keep one table layout
    and clamp every table index, so they stay memory-safe on illegal bytes).
    Fields keep the reference's order, so positional construction means the
    same thing.
    """

    threads: int = LUT23_THREADS
    batch_tile: int = 0
    padded_lut: bool = False
    safe_clamp: bool = False
    k_split: int = 0

    def __post_init__(self) -> None:
        if self.threads <= 0 or self.threads % 32:
            raise FormatError(f"threads must be a positive multiple of the 32-wide simdgroup, got {self.threads}")
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
# The automatic GEMM form may be the wide one above this many activation rows.
WIDE_MIN_AUTO_BATCH = 32


@dataclass(frozen=True)
class GemmConfig:
    """MFMA knobs: the kernel form and the K split (0 = automatic).

    ``form`` picks how weight fragments reach the matrix cores, like the
    reference's ``direct_fragments`` switch (src/ternel_mlx/kernels.py:1043-1188):
    ``"tile"`` decodes 128x128 weight tiles into LDS (prefill), ``"direct"``
    decodes straight into MFMA operand registers (at most 64 activation rows),
    ``"wide"`` decodes into the operand registers of 256-row output tiles (32
    to 256 activation rows wide) split stream-K over the CUs (prefill; K split
    0 or 1), ``"auto"`` takes ``"direct"`` up to 32 rows (48 for matrices under
    16 MiB of packed weights), ``"wide"`` up to 64 and, above, ``"wide"`` when
    it has enough tiles (CUs/4) or work per CU (15 steps) for its stream-K
    reduction to pay, ``"tile"`` otherwise (and, above 32 rows, whenever a K
    split above 1 is fixed).

    The reference's tiling fields (``batch_block`` .. ``safe_clamp``) are
    accepted by keyword so its configurations construct unchanged; they tile
    Apple's 8x8 simdgroup matrices and have no meaning for CDNA4's MFMA, except
    ``direct_fragments``: set (with ``form`` left automatic) it selects the
    direct-fragment form for batches it can hold.
    """

    k_split: int = 0
    form: str = "auto"
    batch_block: int | None = None
    row_block: int | None = None
    k_block: int | None = None
    simd_rows: int | None = None
    simd_columns: int | None = None
    direct_fragments: bool | None = None
    direct_epilogue: bool | None = None
    threadgroup_table: bool | None = None
    safe_clamp: bool = False

    def __post_init__(self) -> None:
        if self.k_split < 0:
            raise FormatError(f"k split must be positive, got {self.k_split}")
        if self.form not in GEMM_FORMS:
            raise FormatError(f"GEMM form must be one of {sorted(GEMM_FORMS)}, got {self.form!r}")
        if self.threadgroup_table and not self.direct_fragments:
            raise FormatError("a threadgroup trit table is only read by the direct-fragment form")

    def form_for(self, batch: int) -> str:
        if self.form == "auto" and self.direct_fragments and batch <= DIRECT_MAX_BATCH:
            return "direct"
        return self.form

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


_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
# Workspaces that a graph may still address: replaced by a larger one after
# their stream was captured, so never freed (a replay would otherwise write
# counters and partials into memory the caching allocator has reused).
_RETIRED: list[torch.Tensor] = []
_CAPTURED: set[tuple[int, int]] = set()


def _aligned_rows(x: torch.Tensor) -> torch.Tensor:
    """``x`` contiguous and 16-byte aligned (the MFMA forms stage activations
    with 16-byte loads): a view at an unaligned storage offset is copied."""
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone(memory_format=torch.contiguous_format)
        if x.data_ptr() % 16:  # the caching allocator's blocks are 512-byte aligned
            raise RuntimeError("could not obtain 16-byte aligned activations")
    return x


def _workspace_key(device: torch.device) -> tuple[int, int]:
    index = device.index if device.index is not None else torch.cuda.current_device()
    return index, torch.cuda.current_stream(torch.device("cuda", index)).cuda_stream


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Zero-initialised split-K scratch, one per (device, stream), grown on demand.

    The kernels leave their counters and piece slots zero after every launch,
    so a buffer only needs zeroing when it is created -- never inside a graph
    capture: size it with an eager call of the same shape first. Calls on one
    stream run in order, so they can share its buffer; calls on two streams
    get two buffers and never race on each other's counters.
    """
    if nbytes == 0:
        return None
    key = _workspace_key(device)
    capturing = torch.cuda.is_current_stream_capturing()
    buf = _WORKSPACES.get(key)
    if capturing and (buf is None or buf.numel() < nbytes):
        # A capture stream (torch.cuda.graph captures on a side stream) borrows
        # the device's largest eager workspace: replays then share it with that
        # stream's eager calls, which must not run at the same time.
        sized = [k for k, b in _WORKSPACES.items() if k[0] == key[0] and b.numel() >= nbytes]
        if not sized:
            raise RuntimeError("split-K workspace must be sized by an eager call before graph capture")
        key = max(sized, key=lambda k: _WORKSPACES[k].numel())
        buf = _WORKSPACES[key]
    if buf is None or buf.numel() < nbytes:
        new = torch.zeros(max(nbytes, 1 << 22), dtype=torch.uint8, device=torch.device("cuda", key[0]))
        torch.cuda.synchronize(key[0])
        if buf is not None and key in _CAPTURED:
            _RETIRED.append(buf)
        _WORKSPACES[key] = buf = new
    if capturing:
        _CAPTURED.add(key)
    return buf


# Launches that may give up a bounded wait (the wide form's stream-K
# reduction) leave an event per workspace; the next call on the device reads
# the error word of every workspace whose event has completed -- no wait on
# the caller's stream, a 4-byte copy on a side stream -- and raises
# ``NativeError`` if it is set, after zeroing that workspace. (The kernels
# themselves refuse a workspace whose word is set: they write the tiles that
# would need its counters as NaN.) Graph replays are not watched; a caller
# replaying graphs runs ``check_workspaces()`` at its own sync points.
_WATCH: dict[tuple[int, int], torch.cuda.Event] = {}
_SIDE: dict[int, torch.cuda.Stream] = {}
_ERROR_WORD_OFFSET = 64 * 1024 - 4  # the last word of the 64 KiB counter region


def _key_of(buf: torch.Tensor) -> tuple[int, int] | None:
    for key, b in _WORKSPACES.items():
        if b is buf:
            return key
    return None


def _watch(ws: torch.Tensor | None, may_give_up: bool) -> None:
    """After a launch: remember to read ``ws``'s error word once it is done."""
    if ws is None or not may_give_up or torch.cuda.is_current_stream_capturing():
        return
    key = _key_of(ws)
    if key is None:
        return
    event = torch.cuda.Event()
    event.record(torch.cuda.current_stream(ws.device))
    _WATCH[key] = event


def _surface(device: torch.device) -> None:
    """Before a launch: raise if a watched workspace of ``device`` reported a
    wait that gave up (zeroing it first, so the next call starts clean)."""
    if not _WATCH or torch.cuda.is_current_stream_capturing():
        return
    index = device.index if device.index is not None else torch.cuda.current_device()
    failed = {}
    for key, event in list(_WATCH.items()):
        if key[0] != index or not event.query():
            continue
        del _WATCH[key]
        buf = _WORKSPACES[key]
        side = _SIDE.get(index)
        if side is None:
            side = _SIDE[index] = torch.cuda.Stream(device=buf.device)
        word = torch.empty(4, dtype=torch.uint8, pin_memory=True)
        with torch.cuda.stream(side):
            side.wait_event(event)
            word.copy_(buf[_ERROR_WORD_OFFSET:_ERROR_WORD_OFFSET + 4], non_blocking=True)
        side.synchronize()
        value = int(word.view(torch.int32).item())
        if value:
            buf.zero_()
            failed[key] = value
    if failed:
        torch.cuda.synchronize(index)
        raise _lib.NativeError(f"a kernel's bounded wait for a published partial gave up: {failed}; "
                               "its tiles were written as NaN and the workspace has been zeroed")


def workspace_errors() -> dict[tuple[int, int], int]:
    """The error word of every workspace (synchronises each one's stream): a
    nonzero word names the kernels whose bounded wait for another workgroup's
    partial gave up (2 = the wide GEMM's stream-K reduction; the LUT23 and
    direct-form fix-ups never wait)."""
    handle = _lib.lib()
    words = {}
    for (index, stream), buf in _WORKSPACES.items():
        word = ctypes.c_int(0)
        with torch.cuda.device(index):
            _lib.check(handle.ternel_tq1_workspace_error(buf.data_ptr(), buf.numel(), ctypes.byref(word), stream))
        words[(index, stream)] = word.value
    return words


def check_workspaces() -> None:
    """Raise ``NativeError`` if any workspace reports a wait that gave up. The
    workspace is zeroed again first (its counters may be left set), so the
    next call starts clean."""
    failed = {key: word for key, word in workspace_errors().items() if word}
    _WATCH.clear()
    for key in failed:
        _WORKSPACES[key].zero_()
    if failed:
        torch.cuda.synchronize()
        raise _lib.NativeError(f"a kernel's bounded wait for a published partial gave up: {failed}")


def tq1_matmul_words(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout,
                     config: MatmulConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` through the LUT23 kernel; ``(batch, rows)`` in ``x.dtype``.
    A ``k_split`` that does not divide the group count is refused, as the
    reference refuses it (src/ternel_mlx/kernels.py:1240-1246)."""
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


def tq1_gemm_words(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout,
                   config: GemmConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` on the MFMA kernels (reference tq1_gemm, kernels.py:1287-1357).

    The matrix cores take fp16 operands (weights are exact in fp16). fp16
    activations run the form ``config`` names; bf16 ones run the wide form,
    each row scaled by a power of two into fp16's range (exact: bf16's
    significand fits fp16's) and the fp32 sums scaled back and rounded once to
    bf16. fp32 activations -- whose significand fp16 would not hold -- and bf16
    ones with a fixed K split run through the LUT23 kernel, which computes in
    fp32 from the activations as given."""
    config = config or GemmConfig()
    check_packed(packed, layout=layout)
    batch = check_activations(x, layout=layout)
    if config.k_split and layout.groups_per_row % config.k_split:
        raise FormatError(
            f"k split {config.k_split} does not divide the tensor's {layout.groups_per_row} groups per row"
        )
    if x.dtype == torch.float32 or (x.dtype == torch.bfloat16 and config.k_split > 1):
        return tq1_matmul_words(packed, x, layout=layout, config=MatmulConfig(batch_tile=1, k_split=config.k_split))
    if x.dtype == torch.bfloat16:
        if config.form not in ("auto", "wide"):
            raise FormatError(f"bf16 activations run the wide GEMM form, not {config.form!r}")
        form_name = "wide"
    else:
        form_name = config.form_for(batch)
    if form_name == "direct" and batch > DIRECT_MAX_BATCH:
        raise FormatError(f"the direct-fragment form takes at most {DIRECT_MAX_BATCH} activation rows, got {batch}")
    form = GEMM_FORMS[form_name]
    x = _aligned_rows(x)
    _surface(x.device)
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    need = handle.ternel_tq1_gemm_workspace_bytes(batch, layout.rows, layout.columns, form, config.k_split)
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_gemm(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns,
        _DTYPE_CODE[x.dtype], form, config.k_split, ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _stream(x.device)))
    _watch(ws, form_name == "wide" or (form_name == "auto" and batch > WIDE_MIN_AUTO_BATCH))
    return out


def tq1_linear_words(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """The library's own dispatch (``ternel_tq1_linear``) for a 2-D ``x``."""
    check_packed(packed, layout=layout)
    batch = check_activations(x, layout=layout)
    x = _aligned_rows(x)
    _surface(x.device)
    out = torch.empty((batch, layout.rows), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    code = _DTYPE_CODE[x.dtype]
    need = handle.ternel_tq1_linear_workspace_bytes(batch, layout.rows, layout.columns, code)
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_linear(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns, code,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(x.device)))
    _watch(ws, handle.ternel_tq1_linear_kernel(batch, layout.rows, layout.columns, code) == GEMM_FORMS["wide"])
    return out


def tq1_swiglu_words(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """SiLU(gate) * up of a SwiGLU MLP whose gate and up projections are one
    packed weight with alternating rows (``layout.interleave_gate_up``):
    ``(batch, rows // 2)`` in ``x.dtype``, each gate/up value rounded to
    ``x.dtype`` as the unfused layers would return it."""
    check_packed(packed, layout=layout)
    batch = check_activations(x, layout=layout)
    if layout.rows % 2:
        raise FormatError(f"a SwiGLU weight interleaves gate and up rows, so its rows must be even, "
                          f"got {layout.rows}")
    x = _aligned_rows(x)
    _surface(x.device)
    out = torch.empty((batch, layout.rows // 2), dtype=x.dtype, device=x.device)
    handle = _lib.lib()
    code = _DTYPE_CODE[x.dtype]
    need = handle.ternel_tq1_swiglu_workspace_bytes(batch, layout.rows, layout.columns, code)
    ws = workspace(x.device, need)
    _lib.check(handle.ternel_tq1_swiglu(
        packed.data_ptr(), x.data_ptr(), out.data_ptr(), batch, layout.rows, layout.columns, code,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(x.device)))
    _watch(ws, handle.ternel_tq1_linear_kernel(batch, layout.rows, layout.columns, code) == GEMM_FORMS["wide"])
    return out


def _gather_ids(indices: torch.Tensor, dtype: torch.dtype, device) -> torch.Tensor:
    if dtype not in ACTIVATION_DTYPES:
        raise FormatError(f"output dtype must be one of {ACTIVATION_DTYPES}, got {dtype}")
    if indices.ndim != 1:
        raise FormatError(f"indices must be 1-D, got shape {tuple(indices.shape)}")
    if indices.numel() <= 0:
        raise FormatError("indices are empty")
    if indices.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8, torch.uint32):
        raise FormatError(f"indices must be an integer tensor, got {indices.dtype}")
    return indices.to(device=device, dtype=torch.int64).contiguous()


def tq1_get_rows_words(packed: torch.Tensor, indices: torch.Tensor, *, layout: PackedTensorLayout,
                       dtype: torch.dtype) -> torch.Tensor:
    """Decode the rows named by ``indices`` (1-D) from packed words; ids outside
    ``[0, rows)`` read as zeros, as the reference kernel does
    (src/ternel_mlx/kernels.py:869-880)."""
    check_packed(packed, layout=layout)
    ids = _gather_ids(indices, dtype, packed.device)
    out = torch.empty((ids.numel(), layout.columns), dtype=dtype, device=packed.device)
    _lib.check(_lib.lib().ternel_tq1_get_rows(
        packed.data_ptr(), layout.rows, layout.columns, ids.data_ptr(), ids.numel(), out.data_ptr(),
        _DTYPE_CODE[dtype], _stream(packed.device)))
    return out


def tq1_get_rows_canonical(blocks: torch.Tensor, indices: torch.Tensor, *, layout: PackedTensorLayout,
                           dtype: torch.dtype) -> torch.Tensor:
    """Row gather over canonical ``(rows, G, 28)`` uint8 device blocks (``unpack_weights``):
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


# ---------------------------------------------------------------------------
# The reference's tiled pair (codes, scales) on the device
# ---------------------------------------------------------------------------
SCALE_DTYPES = (torch.uint16, torch.int16)


def _check_tiled(codes, scales, *, groups_per_row: int, tile: int) -> int:
    """src/ternel_mlx/kernels.py:1191-1212 (same messages), for device tensors."""
    if not isinstance(codes, torch.Tensor) or not isinstance(scales, torch.Tensor):
        raise FormatError("codes and scales must be torch tensors")
    if codes.dtype != torch.uint8:
        raise FormatError(f"codes must be uint8, got {codes.dtype}")
    if scales.dtype not in SCALE_DTYPES:
        raise FormatError(f"scales must be uint16 of raw FP16 bits, got {scales.dtype}")
    if groups_per_row <= 0:
        raise FormatError(f"groups per row must be positive, got {groups_per_row}")
    if tile <= 0:
        raise FormatError(f"tile must be positive, got {tile}")
    if codes.ndim != 4 or tuple(codes.shape[1:]) != (groups_per_row, CODE_SLOTS, tile):
        raise FormatError(
            f"codes shape {tuple(codes.shape)} does not match (tiles, {groups_per_row}, {CODE_SLOTS}, {tile})"
        )
    tiles = codes.shape[0]
    if tuple(scales.shape) != (tiles, groups_per_row, tile):
        raise FormatError(f"scales shape {tuple(scales.shape)} does not match ({tiles}, {groups_per_row}, {tile})")
    if tiles <= 0:
        raise FormatError("packed tensor has no tiles")
    if not codes.is_cuda or not scales.is_cuda or codes.device != scales.device:
        raise FormatError("codes and scales must live on the same GPU")
    return tiles


def _tiled_layout(codes, scales, *, groups_per_row: int, tile: int) -> PackedTensorLayout:
    tiles = _check_tiled(codes, scales, groups_per_row=groups_per_row, tile=tile)
    return PackedTensorLayout(rows=tiles * tile, columns=groups_per_row * BLOCK_SIZE, tile=tile)


def words_from_tiled(codes: torch.Tensor, scales: torch.Tensor, *, layout: PackedTensorLayout,
                     validate: bool = True) -> torch.Tensor:
    """The tiled pair -> packed words on the GPU (exact), scanning every code
    byte on the way; raises the reference's ``validate_packed_codes`` error
    (src/ternel_mlx/packing.py:29-48) when any is out of range."""
    _check_tiled(codes, scales, groups_per_row=layout.groups_per_row, tile=layout.tile)
    codes = codes.contiguous()
    scales = scales.contiguous()
    packed = torch.empty(packed_shape(layout), dtype=torch.int32, device=codes.device)
    counters = torch.empty(2, dtype=torch.int64, device=codes.device)
    _lib.check(_lib.lib().ternel_tq1_words_from_tiled(
        codes.data_ptr(), scales.data_ptr(), layout.rows, layout.columns, layout.tile, packed.data_ptr(),
        counters.data_ptr(), _stream(codes.device)))
    if validate:
        regular, tail = (int(v) for v in counters.cpu())
        if regular or tail:
            from .format import MAX_FULL_CODE_BYTE, MAX_TAIL_CODE_BYTE

            raise FormatError(
                f"packed codes contain out-of-range base-3 bytes: regular={regular} "
                f"(max {MAX_FULL_CODE_BYTE}), tail={tail} (max {MAX_TAIL_CODE_BYTE})"
            )
    return packed


def tiled_from_words(packed: torch.Tensor, *, layout: PackedTensorLayout) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed words -> the reference's ``(codes, scales)`` device tensors (exact)."""
    check_packed(packed, layout=layout)
    codes = torch.empty(layout.codes_shape, dtype=torch.uint8, device=packed.device)
    scales = torch.empty(layout.scales_shape, dtype=torch.uint16, device=packed.device)
    _lib.check(_lib.lib().ternel_tq1_tiled_from_words(
        packed.data_ptr(), layout.rows, layout.columns, layout.tile, codes.data_ptr(), scales.data_ptr(),
        _stream(packed.device)))
    return codes, scales


# Packed words of (codes, scales) pairs the functional calls have seen, keyed by
# the pair's identity and checked against their storage and version counters
# on every hit. An entry goes as soon as either tensor of its pair dies (a
# weakref callback), so a pair's words never outlive it; beyond that the
# cache keeps at most WORD_CACHE_ENTRIES entries and WORD_CACHE_BYTES of words,
# least recently used first out.
WORD_CACHE_ENTRIES = 1024
WORD_CACHE_BYTES = 8 << 30
_WORD_CACHE: OrderedDict[tuple[int, int], tuple] = OrderedDict()
_word_cache_bytes = 0


def _drop_word_entry(key: tuple[int, int], ref: weakref.ref | None = None) -> None:
    """Remove one cache entry (only the one that registered ``ref`` when given:
    a later entry may reuse the key once the first pair's ids are free)."""
    global _word_cache_bytes
    entry = _WORD_CACHE.get(key)
    if entry is None or (ref is not None and entry[0] is not ref and entry[1] is not ref):
        return
    del _WORD_CACHE[key]
    _word_cache_bytes -= entry[3].numel() * entry[3].element_size()


def word_cache_bytes() -> int:
    """Device bytes the functional calls' word cache holds now."""
    return _word_cache_bytes


def words_of(codes: torch.Tensor, scales: torch.Tensor, *, groups_per_row: int, tile: int) -> tuple[
        torch.Tensor, PackedTensorLayout]:
    """Packed words (and layout) for the tiled pair, converted once and cached
    while both tensors live unchanged -- an in-place write bumps a tensor's
    version and forces a new conversion."""
    global _word_cache_bytes
    layout = _tiled_layout(codes, scales, groups_per_row=groups_per_row, tile=tile)
    key = (id(codes), id(scales))
    stamp = (codes.data_ptr(), codes._version, scales.data_ptr(), scales._version, layout)
    hit = _WORD_CACHE.get(key)
    if hit is not None:
        ref_codes, ref_scales, hit_stamp, packed = hit
        if ref_codes() is codes and ref_scales() is scales and hit_stamp == stamp:
            _WORD_CACHE.move_to_end(key)
            return packed, layout
        _drop_word_entry(key)
    packed = words_from_tiled(codes, scales, layout=layout)
    size = packed.numel() * packed.element_size()
    if size > WORD_CACHE_BYTES:
        return packed, layout
    # The callbacks hold only the key and their own weakref: a dead tensor
    # drops its entry without keeping the other one alive.
    ref_codes = weakref.ref(codes, lambda r, key=key: _drop_word_entry(key, r))
    ref_scales = weakref.ref(scales, lambda r, key=key: _drop_word_entry(key, r))
    _WORD_CACHE[key] = (ref_codes, ref_scales, stamp, packed)
    _word_cache_bytes += size
    while len(_WORD_CACHE) > WORD_CACHE_ENTRIES or _word_cache_bytes > WORD_CACHE_BYTES:
        _drop_word_entry(next(iter(_WORD_CACHE)))
    return packed, layout


def _check_activation_width(x: torch.Tensor, *, groups_per_row: int) -> None:
    """src/ternel_mlx/kernels.py:1274-1284, same messages."""
    if x.dtype not in ACTIVATION_DTYPES:
        raise FormatError(f"activations must be one of {ACTIVATION_DTYPES}, got {x.dtype}")
    if x.ndim != 2:
        raise FormatError(f"activations must be 2-D (batch, columns), got shape {tuple(x.shape)}")
    columns = groups_per_row * BLOCK_SIZE
    if x.shape[1] != columns:
        raise FormatError(f"activations have {x.shape[1]} columns, expected {columns}")
    if x.shape[0] <= 0:
        raise FormatError("activations have an empty batch dimension")


def tq1_matmul(codes: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, *, groups_per_row: int, tile: int,
               config: MatmulConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` for a TQ1_G128 packed ``W`` of shape ``(tiles * tile,
    groups_per_row * 128)`` -- the reference's signature and checks
    (src/ternel_mlx/kernels.py:1215-1271). ``x`` is 2-D ``(batch, columns)``;
    the result ``(batch, rows)`` in ``x``'s dtype."""
    config = config or MatmulConfig()
    _check_tiled(codes, scales, groups_per_row=groups_per_row, tile=tile)
    _check_activation_width(x, groups_per_row=groups_per_row)
    if config.k_split and groups_per_row % config.k_split:
        raise FormatError(f"k split {config.k_split} does not divide the tensor's {groups_per_row} groups per row")
    packed, layout = words_of(codes, scales, groups_per_row=groups_per_row, tile=tile)
    return tq1_matmul_words(packed, x, layout=layout, config=config)


def tq1_gemm(codes: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, *, groups_per_row: int, tile: int,
             config: GemmConfig | None = None) -> torch.Tensor:
    """``x @ W.T`` on the matrix cores -- the reference's signature
    (src/ternel_mlx/kernels.py:1287-1357); see ``tq1_gemm_words``."""
    config = config or GemmConfig()
    _check_tiled(codes, scales, groups_per_row=groups_per_row, tile=tile)
    _check_activation_width(x, groups_per_row=groups_per_row)
    packed, layout = words_of(codes, scales, groups_per_row=groups_per_row, tile=tile)
    return tq1_gemm_words(packed, x, layout=layout, config=config)


def tq1_get_rows(codes: torch.Tensor, scales: torch.Tensor, indices: torch.Tensor, *, groups_per_row: int,
                 tile: int, dtype: torch.dtype, threads: int = 256, safe_clamp: bool = False) -> torch.Tensor:
    """Decode the rows named by ``indices`` out of a packed embedding table --
    the reference's signature and checks (src/ternel_mlx/kernels.py:1360-1398).
    ``threads`` is validated as there; ``safe_clamp`` is accepted and has no
    effect (the gather kernel bounds every table access and reads ids outside
    the table as zero rows either way)."""
    _check_tiled(codes, scales, groups_per_row=groups_per_row, tile=tile)
    if dtype not in ACTIVATION_DTYPES:
        raise FormatError(f"output dtype must be one of {ACTIVATION_DTYPES}, got {dtype}")
    if indices.ndim != 1:
        raise FormatError(f"indices must be 1-D, got shape {tuple(indices.shape)}")
    if indices.numel() <= 0:
        raise FormatError("indices are empty")
    if threads <= 0 or threads % 32:
        raise FormatError(f"threads must be a positive multiple of 32, got {threads}")
    packed, layout = words_of(codes, scales, groups_per_row=groups_per_row, tile=tile)
    return tq1_get_rows_words(packed, indices, layout=layout, dtype=dtype)


__all__ = [
    "ACTIVATION_DTYPES",
    "BLOCK_BYTES",
    "GemmConfig",
    "MatmulConfig",
    "check_workspaces",
    "pack_weights",
    "packed_shape",
    "tiled_from_words",
    "tq1_gemm",
    "tq1_gemm_words",
    "tq1_get_rows",
    "tq1_get_rows_canonical",
    "tq1_get_rows_words",
    "tq1_linear_words",
    "tq1_matmul",
    "tq1_matmul_words",
    "tq1_swiglu_words",
    "unpack_weights",
    "words_from_tiled",
    "words_of",
    "workspace_errors",
]
