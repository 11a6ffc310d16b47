"""Tensor geometry and the byte layouts of a packed TQ1_G128 weight.

``PackedTensorLayout`` keeps the reference's API (src/ternel_mlx/layout.py:41-148):
same fields, properties, messages and JSON. Three arrangements of the same
28 bytes per 128 weights exist:

* *canonical* blocks, ``(rows, groups_per_row, 28)`` contiguous -- the bytes
  ``decode_tq1_blocks`` takes and the sidecar stores;
* the reference's *tiled pair* -- ``codes[tile][group][slot][row_in_tile]`` and
  ``scales[tile][group][row_in_tile]`` -- the MLX artifact's arrays and the
  state of its modules; ``pack_blocks``/``unpack_blocks`` convert it on the
  host as src/ternel_mlx/packing.py:51-83 does, ``kernels.words_from_tiled`` /
  ``tiled_from_words`` on the GPU;
* the engine's *packed words* -- what the gfx950 kernels stream: the canonical
  blocks permuted at 4-byte granularity into 64-row tiles, word j of block
  (r, g) at ``packed[r // 64][g][j][r % 64]`` (uint32), rows past the end zero,
  so one wave64 reads one word of 64 rows' blocks with one coalesced 256-byte
  load (``kernels.pack_weights`` / ``unpack_weights``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .format import BLOCK_BYTES, BLOCK_SIZE, CODE_SLOTS, FormatError

LAYOUT_VERSION = 1
LAYOUT_NAME = "TQ1_G128_MLX_TILED"
DEVICE_LAYOUT_NAME = "TQ1_G128_WORDS_64_ROW_INTERLEAVED"
PREFERRED_TILE = 256
SCALE_BYTES = BLOCK_BYTES - CODE_SLOTS
CODES_SUFFIX = "codes"
SCALES_SUFFIX = "scales"
SCALE_VIEW_DTYPE = np.dtype("<u2")


def select_tile(rows: int) -> int:
    """256 when it divides ``rows``, else ``rows`` (src/ternel_mlx/layout.py:41-51)."""
    if rows <= 0:
        raise FormatError(f"row count must be positive, got {rows}")
    if rows % PREFERRED_TILE == 0:
        return PREFERRED_TILE
    return rows


@dataclass(frozen=True)
class PackedTensorLayout:
    """Shape and byte accounting of one packed tensor (src/ternel_mlx/layout.py:54-148).

    ``rows`` is the output dimension, ``columns`` the reduction dimension.
    """

    rows: int
    columns: int
    tile: int

    def __post_init__(self) -> None:
        if self.rows <= 0 or self.columns <= 0:
            raise FormatError(f"tensor dimensions must be positive, got {self.rows}x{self.columns}")
        if self.columns % BLOCK_SIZE:
            raise FormatError(
                f"{self.columns} columns is not a multiple of the {BLOCK_SIZE}-weight group"
            )
        if self.tile <= 0:
            raise FormatError(f"tile must be positive, got {self.tile}")
        if self.rows % self.tile:
            raise FormatError(
                f"tile {self.tile} does not divide {self.rows} rows; the MLX layout does not pad rows"
            )

    @classmethod
    def for_tensor(cls, rows: int, columns: int) -> "PackedTensorLayout":
        return cls(rows=rows, columns=columns, tile=select_tile(rows))

    @property
    def groups_per_row(self) -> int:
        return self.columns // BLOCK_SIZE

    @property
    def tiles(self) -> int:
        return self.rows // self.tile

    @property
    def groups(self) -> int:
        return self.rows * self.groups_per_row

    @property
    def codes_shape(self) -> tuple[int, int, int, int]:
        return (self.tiles, self.groups_per_row, CODE_SLOTS, self.tile)

    @property
    def scales_shape(self) -> tuple[int, int, int]:
        return (self.tiles, self.groups_per_row, self.tile)

    @property
    def canonical_shape(self) -> tuple[int, int, int]:
        """Device layout of this engine: ``(rows, groups_per_row, 28)`` uint8."""
        return (self.rows, self.groups_per_row, BLOCK_BYTES)

    @property
    def codes_bytes(self) -> int:
        return self.groups * CODE_SLOTS

    @property
    def scales_bytes(self) -> int:
        return self.groups * SCALE_BYTES

    @property
    def payload_bytes(self) -> int:
        return self.codes_bytes + self.scales_bytes

    @property
    def canonical_bytes(self) -> int:
        return self.groups * BLOCK_BYTES

    @property
    def bits_per_weight(self) -> float:
        return self.payload_bytes * 8 / (self.rows * self.columns)

    def to_json(self) -> dict[str, object]:
        return {
            "layout_name": LAYOUT_NAME,
            "layout_version": LAYOUT_VERSION,
            "rows": self.rows,
            "columns": self.columns,
            "tile": self.tile,
            "tiles": self.tiles,
            "groups_per_row": self.groups_per_row,
            "groups": self.groups,
            "codes_shape": list(self.codes_shape),
            "scales_shape": list(self.scales_shape),
            "codes_bytes": self.codes_bytes,
            "scales_bytes": self.scales_bytes,
            "payload_bytes": self.payload_bytes,
            "bits_per_weight": self.bits_per_weight,
        }


def pack_blocks(blocks: np.ndarray, *, layout: PackedTensorLayout) -> tuple[np.ndarray, np.ndarray]:
    """Canonical ``(rows, G, 28)`` -> ``(codes u8, scales <u2)`` (src/ternel_mlx/packing.py:51-64)."""
    source = np.asarray(blocks)
    if source.dtype != np.uint8:
        raise FormatError(f"canonical blocks must be uint8, got {source.dtype}")
    if source.shape != layout.canonical_shape:
        raise FormatError(f"expected canonical blocks of shape {layout.canonical_shape}, got {source.shape}")
    t, g, tile = layout.tiles, layout.groups_per_row, layout.tile
    tiled = source.reshape(t, tile, g, BLOCK_BYTES)
    codes = np.ascontiguousarray(tiled[:, :, :, 2:].transpose(0, 2, 3, 1))
    scale_pairs = np.ascontiguousarray(tiled[:, :, :, :2].transpose(0, 2, 1, 3))
    scales = scale_pairs.reshape(-1).view(SCALE_VIEW_DTYPE).reshape(layout.scales_shape)
    return codes, scales


def unpack_blocks(codes: np.ndarray, scales: np.ndarray, *, layout: PackedTensorLayout) -> np.ndarray:
    """Inverse of :func:`pack_blocks` (src/ternel_mlx/packing.py:67-82)."""
    code_array = np.asarray(codes)
    scale_array = np.asarray(scales)
    if code_array.dtype != np.uint8:
        raise FormatError(f"codes must be uint8, got {code_array.dtype}")
    if scale_array.dtype != SCALE_VIEW_DTYPE:
        raise FormatError(f"scales must be little-endian uint16, got {scale_array.dtype}")
    if code_array.shape != layout.codes_shape:
        raise FormatError(f"codes shape {code_array.shape} does not match {layout.codes_shape}")
    if scale_array.shape != layout.scales_shape:
        raise FormatError(f"scales shape {scale_array.shape} does not match {layout.scales_shape}")
    t, g, tile = layout.tiles, layout.groups_per_row, layout.tile
    out = np.empty((t, tile, g, BLOCK_BYTES), dtype=np.uint8)
    out[:, :, :, 2:] = code_array.transpose(0, 3, 1, 2)
    pairs = np.ascontiguousarray(scale_array).reshape(-1).view(np.uint8).reshape(t, g, tile, 2)
    out[:, :, :, :2] = pairs.transpose(0, 2, 1, 3)
    return out.reshape(layout.canonical_shape)


def interleave_gate_up(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """Canonical blocks of a SwiGLU MLP's gate and up projections, (rows, G, 28)
    each, as one ``(2 rows, G, 28)`` weight whose rows alternate gate, up: row
    2r is gate row r and row 2r + 1 up row r, the order the fused SwiGLU
    epilogue pairs them in."""
    g, u = np.asarray(gate), np.asarray(up)
    if g.dtype != np.uint8 or u.dtype != np.uint8:
        raise FormatError("gate and up blocks must be uint8")
    if g.shape != u.shape or g.ndim != 3 or g.shape[2] != BLOCK_BYTES:
        raise FormatError(f"gate {g.shape} and up {u.shape} must be canonical blocks of one shape")
    return np.stack([g, u], axis=1).reshape(2 * g.shape[0], g.shape[1], BLOCK_BYTES)


@dataclass(frozen=True)
class ModelLinearShape:
    """One distinct linear shape of Ternary Bonsai 27B (src/ternel_mlx/layout.py:151-176)."""

    label: str
    rows: int
    columns: int
    dispatches_per_token: int
    modules: tuple[str, ...]

    def layout(self) -> PackedTensorLayout:
        return PackedTensorLayout.for_tensor(self.rows, self.columns)


# Census of src/ternel_mlx/layout.py:179-192 (shapes and per-token dispatch counts).
MODEL_LINEAR_SHAPES: tuple[ModelLinearShape, ...] = (
    ModelLinearShape("linear_attn.in_proj_a", 48, 5120, 96, ("linear_attn.in_proj_a", "linear_attn.in_proj_b")),
    ModelLinearShape("self_attn.k_proj", 1024, 5120, 32, ("self_attn.k_proj", "self_attn.v_proj")),
    ModelLinearShape("linear_attn.out_proj", 5120, 6144, 64, ("linear_attn.out_proj", "self_attn.o_proj")),
    ModelLinearShape("mlp.down_proj", 5120, 17408, 64, ("mlp.down_proj",)),
    ModelLinearShape("linear_attn.in_proj_z", 6144, 5120, 48, ("linear_attn.in_proj_z",)),
    ModelLinearShape("linear_attn.in_proj_qkv", 10240, 5120, 48, ("linear_attn.in_proj_qkv",)),
    ModelLinearShape("self_attn.q_proj", 12288, 5120, 16, ("self_attn.q_proj",)),
    ModelLinearShape("mlp.gate_proj", 17408, 5120, 128, ("mlp.gate_proj", "mlp.up_proj")),
    ModelLinearShape("lm_head", 248320, 5120, 1, ("lm_head",)),
)
DISPATCHES_PER_TOKEN = 497

if sum(shape.dispatches_per_token for shape in MODEL_LINEAR_SHAPES) != DISPATCHES_PER_TOKEN:
    raise FormatError("the shape census no longer accounts for a whole decoded token")
