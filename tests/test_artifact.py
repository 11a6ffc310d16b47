"""Host side of the artifact loaders: the sidecar header and manifest checks of
tests/test_format.py:116-143,193-272 (same fixtures, mutations and messages),
write -> read round trips, and the MLX safetensors pair by exact permutation."""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from oracle import tq1_oracle as O
from ternel_amd.artifact import (
    HEADER_BYTES,
    SidecarHeader,
    align_up,
    canonical_json_bytes,
    read_sidecar,
    safetensors_blocks,
    safetensors_layout,
    save_safetensors,
    sidecar_blocks,
    sidecar_tensors,
    write_sidecar,
)
from ternel_amd.format import FormatError


def random_blocks(rows: int, groups: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    scales = rng.integers(0, 256, size=(rows * groups, 2), dtype=np.uint8)
    trits = rng.integers(0, 3, size=(rows * groups, 128), dtype=np.uint8)
    return O.encode_tq1_blocks(scales, trits).reshape(rows, groups, 28)


def test_header_round_trip_and_reserved_bytes() -> None:
    header = SidecarHeader(version=1, header_bytes=256, block_size=128, block_bytes=28, alignment=256,
                           tensor_count=2, source_file_bytes=1234, manifest_offset=4096, manifest_bytes=987,
                           source_sha256="12" * 32)
    encoded = header.pack()
    assert len(encoded) == HEADER_BYTES
    assert encoded[:8] == b"TQ1G128\0"
    assert encoded[88:] == bytes(HEADER_BYTES - 88)
    # little-endian fields at the reference's offsets
    assert struct.unpack_from("<IIIIII", encoded, 8) == (1, 256, 128, 28, 256, 2)
    assert struct.unpack_from("<QQQ", encoded, 32) == (1234, 4096, 987)
    assert encoded[56:88] == bytes.fromhex("12" * 32)
    assert SidecarHeader.unpack(encoded) == header


def test_header_rejects_nonhex_hash_and_nonzero_reserved_byte() -> None:
    with pytest.raises(FormatError, match="hexadecimal"):
        SidecarHeader(1, 256, 128, 28, 256, 0, 0, 256, 2, "z" * 64).pack()
    with pytest.raises(FormatError, match="64 hexadecimal"):
        SidecarHeader(1, 256, 128, 28, 256, 0, 0, 256, 2, "ab").pack()
    corrupted = bytearray(SidecarHeader(1, 256, 128, 28, 256, 0, 0, 256, 2, "00" * 32).pack())
    corrupted[-1] = 1
    with pytest.raises(FormatError, match="reserved"):
        SidecarHeader.unpack(corrupted)
    with pytest.raises(FormatError, match="truncated"):
        SidecarHeader.unpack(bytes(100))


def _sidecar_bytes() -> bytes:
    """The reference's two-tensor fixture (tests/test_format.py:193-215)."""
    tensors = [
        {"name": "a", "packed_offset": 256, "packed_bytes": 56, "groups": 2},
        {"name": "b", "packed_offset": 512, "packed_bytes": 28, "groups": 1},
    ]
    manifest = canonical_json_bytes({"format": "TQ1_G128", "tensors": tensors})
    header = SidecarHeader(1, 256, 128, 28, 256, 2, 999, 540, len(manifest), "ab" * 32)
    data = bytearray(header.pack())
    data.extend(bytes(540 - len(data)))
    data.extend(manifest)
    return bytes(data)


def test_read_sidecar_accepts_valid_aligned_tensor_extents(tmp_path) -> None:
    path = tmp_path / "valid.tq1"
    path.write_bytes(_sidecar_bytes())
    header, manifest = read_sidecar(path)
    assert header.tensor_count == 2
    assert [t["name"] for t in manifest["tensors"]] == ["a", "b"]


@pytest.mark.parametrize(("mutation", "message"), [
    ("magic", "magic"),
    ("version", "version"),
    ("geometry", "geometry"),
    ("manifest_bounds", "outside"),
    ("manifest_json", "manifest"),
    ("manifest_format", "format"),
    ("tensor_count", "tensor count"),
    ("unaligned_tensor", "extent"),
    ("wrong_tensor_size", "extent"),
    ("overlap_manifest", "overlaps"),
])
def test_read_sidecar_rejects_corruption(tmp_path, mutation: str, message: str) -> None:
    data = bytearray(_sidecar_bytes())
    header = SidecarHeader.unpack(bytes(data[:HEADER_BYTES]))
    manifest = json.loads(data[header.manifest_offset:].decode())
    if mutation == "magic":
        data[0] ^= 0xFF
    elif mutation == "version":
        struct.pack_into("<I", data, 8, 99)
    elif mutation == "geometry":
        struct.pack_into("<I", data, 16, 127)
    elif mutation == "manifest_bounds":
        struct.pack_into("<Q", data, 48, len(data) + 1)
    elif mutation == "manifest_json":
        data[header.manifest_offset] = 0xFF
    else:
        if mutation == "manifest_format":
            manifest["format"] = "wrong"
        elif mutation == "tensor_count":
            manifest["tensors"].pop()
        elif mutation == "unaligned_tensor":
            manifest["tensors"][1]["packed_offset"] = 511
        elif mutation == "wrong_tensor_size":
            manifest["tensors"][0]["packed_bytes"] = 55
        elif mutation == "overlap_manifest":
            manifest["tensors"][1]["packed_bytes"] = 56
            manifest["tensors"][1]["groups"] = 2
        replacement = canonical_json_bytes(manifest)
        data = data[:header.manifest_offset] + replacement
        struct.pack_into("<Q", data, 48, len(replacement))
    path = tmp_path / f"{mutation}.tq1"
    path.write_bytes(bytes(data))
    with pytest.raises(FormatError, match=message):
        read_sidecar(path)


@pytest.mark.parametrize("alignment", (0, -1, 3, 6))
def test_align_up_rejects_non_power_of_two(alignment: int) -> None:
    with pytest.raises(ValueError, match="power of two"):
        align_up(10, alignment)


def test_align_up_rounds_to_the_next_multiple() -> None:
    assert [align_up(v) for v in (0, 1, 255, 256, 257)] == [0, 256, 256, 256, 512]
    assert align_up(10, 8) == 16


def test_written_sidecar_round_trips_every_block(tmp_path) -> None:
    tensors = {"blk.0.ffn_down.weight": random_blocks(300, 5, seed=1),
               "blk.0.attn_q.weight": random_blocks(64, 3, seed=2),
               "token_embd.weight": random_blocks(7, 1, seed=3)}
    path = tmp_path / "model.tq1"
    header = write_sidecar(path, tensors, source_sha256="cd" * 32, source_file_bytes=12345)
    read_header, manifest = read_sidecar(path)
    assert read_header == header
    assert manifest["format"] == "TQ1_G128" and manifest["mapping"] == {"-1": 0, "0": 1, "+1": 2}
    entries = sidecar_tensors(manifest)
    assert list(entries) == list(tensors)
    for name, blocks in tensors.items():
        entry = entries[name]
        assert (entry.rows, entry.columns) == (blocks.shape[0], blocks.shape[1] * 128)
        assert entry.offset % 256 == 0
        np.testing.assert_array_equal(np.asarray(sidecar_blocks(path, entry)), blocks)
    # payloads sit where the manifest says, padding in between is zero
    raw = path.read_bytes()
    assert raw[:HEADER_BYTES] == header.pack()
    first = entries["blk.0.ffn_down.weight"]
    assert raw[first.offset:first.offset + first.nbytes] == tensors["blk.0.ffn_down.weight"].tobytes()


def test_manifest_shapes_must_describe_2d_weights(tmp_path) -> None:
    path = tmp_path / "model.tq1"
    write_sidecar(path, {"w": random_blocks(4, 2, seed=4)})
    _, manifest = read_sidecar(path)
    manifest["tensors"][0]["shape_gguf"] = [256, 3]
    with pytest.raises(FormatError, match="not a 2-D weight"):
        sidecar_tensors(manifest)


@pytest.mark.parametrize(("rows", "groups"), ((512, 3), (300, 2), (256, 1), (1, 4)))
def test_safetensors_pair_round_trips_by_exact_permutation(tmp_path, rows: int, groups: int) -> None:
    blocks = random_blocks(rows, groups, seed=rows + groups)
    path = tmp_path / "model.safetensors"
    save_safetensors(path, {"model.layers.0.mlp.down_proj": blocks})
    layout, back = safetensors_blocks(path, "model.layers.0.mlp.down_proj")
    assert (layout.rows, layout.columns) == (rows, groups * 128)
    assert layout.tile == (256 if rows % 256 == 0 else rows)
    np.testing.assert_array_equal(back, blocks)


def test_safetensors_pair_with_an_illegal_tile_is_rejected() -> None:
    # 512 rows must be two tiles of 256, not one of 512
    with pytest.raises(FormatError, match="tile rule"):
        safetensors_layout((1, 2, 26, 512), (1, 2, 512))
    with pytest.raises(FormatError, match="not a packed pair"):
        safetensors_layout((2, 26, 256), (1, 2, 256))


def test_missing_tensor_names_are_reported(tmp_path) -> None:
    path = tmp_path / "model.safetensors"
    save_safetensors(path, {"a": random_blocks(4, 1, seed=9)})
    with pytest.raises(FormatError, match="no packed tensor 'b'"):
        safetensors_blocks(path, "b")


def test_interleave_gate_up_alternates_rows() -> None:
    from ternel_amd.layout import interleave_gate_up

    gate, up = random_blocks(5, 2, seed=20), random_blocks(5, 2, seed=21)
    fused = interleave_gate_up(gate, up)
    assert fused.shape == (10, 2, 28)
    np.testing.assert_array_equal(fused[0::2], gate)
    np.testing.assert_array_equal(fused[1::2], up)
    with pytest.raises(FormatError, match="one shape"):
        interleave_gate_up(gate, up[:4])
