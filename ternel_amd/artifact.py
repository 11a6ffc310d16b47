"""TQ1_G128 weights from the reference's two on-disk artifacts, onto the GPU.

* The canonical sidecar (src/bonsai_tq1/format.py:150-246; written by
  src/bonsai_tq1/pack_model.py:50-150): a 256-byte header (magic
  ``TQ1G128\\0``, version, geometry, tensor count, source size, manifest extent,
  source SHA-256; the rest zero), each tensor's canonical 28-byte blocks at a
  256-byte-aligned offset in GGUF row order, and a canonical-JSON manifest
  after the last tensor.
* The MLX safetensors artifact (src/ternel_mlx/layout.py:37-38,
  src/ternel_mlx/packing.py:51-83): per packed tensor ``<name>.codes`` (u8,
  ``(tiles, G, 26, tile)``) and ``<name>.scales`` (u16 raw fp16 bits,
  ``(tiles, G, tile)``), with ``tile = 256`` when it divides the rows and the
  row count otherwise, so the tiled shape gives the rows exactly.

Both are read on the host without executing anything from the file (struct,
JSON, memory map, safetensors), land on the GPU as canonical blocks, are
scanned there for out-of-range code bytes (fail-closed, the reference's
load-time check) and are permuted into the packed words the kernels read.
Header and manifest checks raise :class:`FormatError` with the reference's
messages.
"""

from __future__ import annotations

import hashlib
import json
import struct
import warnings
from dataclasses import dataclass
from pathlib import Path
from typing import Mapping

import numpy as np
import torch

from .format import BLOCK_BYTES, BLOCK_SIZE, FormatError, as_device_blocks, validate_packed_codes
from .layout import SCALE_VIEW_DTYPE, PackedTensorLayout, pack_blocks, select_tile, unpack_blocks

# Sidecar geometry (src/bonsai_tq1/format.py:14-30).
HEADER_BYTES = 256
ALIGNMENT = 256
MAGIC = b"TQ1G128\0"
VERSION = 1
# magic, version, header bytes, block size, block bytes, alignment, tensor
# count (u32 each after the magic), source file bytes, manifest offset,
# manifest bytes (u64), source SHA-256 (32 raw bytes): 88 bytes, little-endian.
HEADER_STRUCT = struct.Struct("<8sIIIIIIQQQ32s")
MANIFEST_FORMAT = "TQ1_G128"
CODES_SUFFIX = "codes"
SCALES_SUFFIX = "scales"


def align_up(value: int, alignment: int = ALIGNMENT) -> int:
    """Round up to a power-of-two alignment (src/bonsai_tq1/format.py:37-40)."""
    if alignment <= 0 or alignment & (alignment - 1):
        raise ValueError("alignment must be a positive power of two")
    return -(-value // alignment) * alignment


def canonical_json_bytes(value: object) -> bytes:
    """Sorted keys, no whitespace, UTF-8 (src/bonsai_tq1/format.py:261-262)."""
    return json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=False).encode("utf-8")


@dataclass(frozen=True)
class SidecarHeader:
    """The sidecar's fixed header (src/bonsai_tq1/format.py:150-218)."""

    version: int
    header_bytes: int
    block_size: int
    block_bytes: int
    alignment: int
    tensor_count: int
    source_file_bytes: int
    manifest_offset: int
    manifest_bytes: int
    source_sha256: str

    def pack(self) -> bytes:
        if len(self.source_sha256) != 64:
            raise FormatError("source SHA-256 must contain 64 hexadecimal characters")
        try:
            digest = bytes.fromhex(self.source_sha256)
        except ValueError as exc:
            raise FormatError("source SHA-256 is not hexadecimal") from exc
        fields = HEADER_STRUCT.pack(MAGIC, self.version, self.header_bytes, self.block_size, self.block_bytes,
                                    self.alignment, self.tensor_count, self.source_file_bytes,
                                    self.manifest_offset, self.manifest_bytes, digest)
        return fields.ljust(HEADER_BYTES, b"\0")

    @classmethod
    def unpack(cls, data: bytes) -> "SidecarHeader":
        if len(data) < HEADER_BYTES:
            raise FormatError("truncated TQ1 header")
        if any(bytes(data[HEADER_STRUCT.size:HEADER_BYTES])):
            raise FormatError("nonzero reserved TQ1 header bytes")
        magic, *numbers, digest = HEADER_STRUCT.unpack_from(bytes(data[:HEADER_STRUCT.size]))
        if magic != MAGIC:
            raise FormatError("invalid TQ1 magic")
        header = cls(*numbers, source_sha256=digest.hex())
        if header.version != VERSION:
            raise FormatError(f"unsupported TQ1 version {header.version}")
        geometry = (header.header_bytes, header.block_size, header.block_bytes, header.alignment)
        if geometry != (HEADER_BYTES, BLOCK_SIZE, BLOCK_BYTES, ALIGNMENT):
            raise FormatError("unsupported TQ1 geometry")
        return header


@dataclass(frozen=True)
class SidecarTensor:
    """One manifest entry, with the logical shape the kernels use."""

    name: str
    rows: int     # output dimension (GGUF ne1)
    columns: int  # reduction dimension (GGUF ne0)
    offset: int
    nbytes: int

    @property
    def layout(self) -> PackedTensorLayout:
        return PackedTensorLayout.for_tensor(self.rows, self.columns)


def read_sidecar(path) -> tuple[SidecarHeader, dict]:
    """Header and manifest, every extent checked (src/bonsai_tq1/format.py:221-246)."""
    path = Path(path)
    size = path.stat().st_size
    with path.open("rb") as handle:
        header = SidecarHeader.unpack(handle.read(HEADER_BYTES))
        if header.manifest_offset < HEADER_BYTES or header.manifest_offset + header.manifest_bytes > size:
            raise FormatError("manifest points outside the sidecar")
        handle.seek(header.manifest_offset)
        raw = handle.read(header.manifest_bytes)
    try:
        manifest = json.loads(raw)
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise FormatError("invalid sidecar manifest") from exc
    if not isinstance(manifest, dict) or manifest.get("format") != MANIFEST_FORMAT:
        raise FormatError("unexpected sidecar manifest format")
    entries = manifest.get("tensors")
    if not isinstance(entries, list) or len(entries) != header.tensor_count:
        raise FormatError("sidecar tensor count does not match manifest")
    end = HEADER_BYTES
    for entry in entries:
        offset, nbytes, groups = int(entry["packed_offset"]), int(entry["packed_bytes"]), int(entry["groups"])
        if offset % ALIGNMENT or offset < align_up(end) or nbytes != groups * BLOCK_BYTES:
            raise FormatError(f"invalid tensor extent for {entry.get('name', '<unknown>')}")
        if offset + nbytes > header.manifest_offset:
            raise FormatError("tensor data overlaps the manifest")
        end = offset + nbytes
    return header, manifest


def sidecar_tensors(manifest: dict) -> dict[str, SidecarTensor]:
    """Manifest entries by name. ``shape_gguf`` is (columns, rows): GGUF lists
    the contiguous dimension first."""
    out: dict[str, SidecarTensor] = {}
    for entry in manifest["tensors"]:
        name = str(entry["name"])
        shape = [int(d) for d in entry.get("shape_gguf", ())]
        groups = int(entry["groups"])
        if len(shape) != 2 or shape[0] % BLOCK_SIZE or shape[0] * shape[1] != groups * BLOCK_SIZE:
            raise FormatError(f"tensor {name} has shape {shape}, not a 2-D weight of {groups} groups")
        out[name] = SidecarTensor(name, rows=shape[1], columns=shape[0], offset=int(entry["packed_offset"]),
                                  nbytes=int(entry["packed_bytes"]))
    return out


def sidecar_blocks(path, tensor: SidecarTensor) -> np.ndarray:
    """Read-only memory map of one tensor's canonical blocks, (rows, G, 28)."""
    layout = tensor.layout
    return np.memmap(Path(path), mode="r", dtype=np.uint8, offset=tensor.offset, shape=layout.canonical_shape)


def write_sidecar(path, tensors: Mapping[str, np.ndarray], *, source_sha256: str = "0" * 64,
                  source_file_bytes: int = 0) -> SidecarHeader:
    """Write canonical ``(rows, G, 28)`` blocks as a sidecar the reference's
    ``read_sidecar`` accepts: payloads at 256-byte-aligned offsets in the given
    order, then the manifest, with the header written last."""
    path = Path(path)
    entries = []
    offset = HEADER_BYTES
    arrays = []
    for name, blocks in tensors.items():
        array = np.ascontiguousarray(np.asarray(blocks, dtype=np.uint8))
        if array.ndim != 3 or array.shape[2] != BLOCK_BYTES:
            raise FormatError(f"tensor {name}: expected canonical blocks (rows, G, 28), got {array.shape}")
        rows, groups_per_row = array.shape[:2]
        offset = align_up(offset)
        entries.append({
            "name": name,
            "shape_gguf": [groups_per_row * BLOCK_SIZE, rows],
            "elements": rows * groups_per_row * BLOCK_SIZE,
            "groups": rows * groups_per_row,
            "packed_offset": offset,
            "packed_bytes": array.nbytes,
            "packed_payload_sha256": hashlib.sha256(array.tobytes()).hexdigest(),
        })
        arrays.append((offset, array))
        offset += array.nbytes
    manifest = canonical_json_bytes({
        "format": MANIFEST_FORMAT,
        "version": VERSION,
        "block_size": BLOCK_SIZE,
        "block_bytes": BLOCK_BYTES,
        "alignment": ALIGNMENT,
        "mapping": {"-1": 0, "0": 1, "+1": 2},
        "packed_payload_bytes": sum(entry["packed_bytes"] for entry in entries),
        "tensors": entries,
    })
    header = SidecarHeader(VERSION, HEADER_BYTES, BLOCK_SIZE, BLOCK_BYTES, ALIGNMENT, len(entries),
                           source_file_bytes, offset, len(manifest), source_sha256)
    packed_header = header.pack()
    with path.open("wb") as handle:
        handle.write(bytes(HEADER_BYTES))
        for start, array in arrays:
            handle.write(bytes(start - handle.tell()))
            handle.write(array.tobytes())
        handle.write(manifest)
        handle.seek(0)
        handle.write(packed_header)
    return header


def upload(blocks, layout: PackedTensorLayout, *, device=None, validate: bool = True) -> torch.Tensor:
    """Canonical blocks (host or device) -> the packed words the kernels read,
    after the full on-GPU scan of every code byte."""
    from .kernels import pack_weights

    if not isinstance(blocks, torch.Tensor):
        # A read-only memory map: torch warns about wrapping it, but the host
        # tensor is only the source of the device copy and is never written.
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)
            host = torch.from_numpy(np.ascontiguousarray(blocks, dtype=np.uint8))
        blocks = host.to(device) if device is not None else host
    tensor = as_device_blocks(blocks)
    if tensor.shape[0] != layout.groups:
        raise FormatError(f"expected {layout.groups} blocks for {layout.rows}x{layout.columns}, "
                          f"got {tensor.shape[0]}")
    if validate:
        validate_packed_codes(tensor)
    return pack_weights(tensor, layout=layout)


def load_sidecar_tensor(path, name: str, *, device=None, validate: bool = True):
    """``(layout, packed words)`` of one sidecar tensor."""
    _, manifest = read_sidecar(path)
    tensors = sidecar_tensors(manifest)
    if name not in tensors:
        raise FormatError(f"sidecar has no tensor {name!r}")
    tensor = tensors[name]
    return tensor.layout, upload(sidecar_blocks(path, tensor), tensor.layout, device=device, validate=validate)


def safetensors_layout(codes_shape, scales_shape) -> PackedTensorLayout:
    """The layout a tiled ``codes`` / ``scales`` pair encodes: tiles x tile rows."""
    if len(codes_shape) != 4 or len(scales_shape) != 3:
        raise FormatError(f"codes {tuple(codes_shape)} / scales {tuple(scales_shape)} are not a packed pair")
    tiles, groups_per_row, slots, tile = (int(d) for d in codes_shape)
    rows = tiles * tile
    layout = PackedTensorLayout.for_tensor(rows, groups_per_row * BLOCK_SIZE)
    if select_tile(rows) != tile or tuple(codes_shape) != layout.codes_shape or \
            tuple(scales_shape) != layout.scales_shape:
        raise FormatError(f"codes {tuple(codes_shape)} / scales {tuple(scales_shape)} do not match the tile "
                          f"rule for {rows} rows")
    return layout


def safetensors_blocks(path, name: str) -> tuple[PackedTensorLayout, np.ndarray]:
    """Canonical blocks of ``<name>.codes`` / ``<name>.scales`` (exact inverse
    permutation, src/ternel_mlx/packing.py:67-83)."""
    from safetensors import safe_open

    with safe_open(str(path), framework="numpy") as handle:
        keys = set(handle.keys())
        codes_key, scales_key = f"{name}.{CODES_SUFFIX}", f"{name}.{SCALES_SUFFIX}"
        if codes_key not in keys or scales_key not in keys:
            raise FormatError(f"{path} has no packed tensor {name!r}")
        codes = handle.get_tensor(codes_key)
        scales = handle.get_tensor(scales_key)
    if scales.dtype in (np.int16, np.uint16):
        scales = scales.view(SCALE_VIEW_DTYPE)
    layout = safetensors_layout(codes.shape, scales.shape)
    return layout, unpack_blocks(codes, scales, layout=layout)


def load_safetensors_tensor(path, name: str, *, device=None, validate: bool = True):
    """``(layout, packed words)`` of one MLX-artifact tensor."""
    layout, blocks = safetensors_blocks(path, name)
    return layout, upload(blocks, layout, device=device, validate=validate)


def save_safetensors(path, tensors: Mapping[str, np.ndarray]) -> None:
    """Write canonical blocks as the MLX artifact's tiled pairs (for tests and
    for converting weights this engine packed)."""
    from safetensors.numpy import save_file

    arrays = {}
    for name, blocks in tensors.items():
        array = np.asarray(blocks, dtype=np.uint8)
        layout = PackedTensorLayout.for_tensor(array.shape[0], array.shape[1] * BLOCK_SIZE)
        codes, scales = pack_blocks(array, layout=layout)
        arrays[f"{name}.{CODES_SUFFIX}"] = codes
        arrays[f"{name}.{SCALES_SUFFIX}"] = np.ascontiguousarray(scales).view(np.uint16)
    save_file(arrays, str(path))


__all__ = [
    "ALIGNMENT", "HEADER_BYTES", "HEADER_STRUCT", "MAGIC", "VERSION", "SidecarHeader", "SidecarTensor",
    "align_up", "canonical_json_bytes", "load_safetensors_tensor", "load_sidecar_tensor", "read_sidecar",
    "safetensors_blocks", "safetensors_layout", "save_safetensors", "sidecar_blocks", "sidecar_tensors", "upload",
    "write_sidecar",
]
