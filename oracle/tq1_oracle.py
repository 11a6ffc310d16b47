"""CPU oracle for the TQ1_G128 packed-weight path -- TEST INFRASTRUCTURE ONLY.

This module restates, in plain numpy, the reference's CPU algorithms for the
hot path so that the HIP kernels can be checked against them. It is never the
thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker.
The product path (``ternel_amd``) never imports this file.

Every function names the reference file:line it follows (paths are relative to
the reference repository root, ``inductiveML/ternel``).

How each function is pinned (so that a plausible mistake fails a check):

* ``decode_tq1_blocks`` / ``count_invalid`` -- against the closed-form truth
  table of all 256 byte values (``tests/golden/decode_truth_table.npz``, built by
  repeated integer division in pure Python), the reference's known-answer tests
  (byte 243 -> ``regular=1``, tail 27 -> ``tail=1``, every legal byte and tail
  byte round-trips, all 65,536 scale patterns survive), and planted mistakes.
* ``encode_tq1_blocks`` -- inverse of the truth table + round trip.
* ``decode_q2_blocks`` -- the reference's known answer (codes 0,1,2,3 repeated
  with scale bytes 0xAA 0x55 decode in that order, tests/test_format.py:94-102),
  a bit-by-bit pure-Python restatement over all 256 byte values at every
  position, and the Q2 and TQ1 reference GEMVs agreeing exactly after
  repacking (tests/test_format.py:146-158).
* ``reorder_tensor_arrays`` / ``restore_tensor_arrays`` -- index formula on
  brute-force loops + round trip at rows {1, 48, 256, 257, 513}.
* ``reference_gemv`` / ``lut23_matmul`` / ``oracle_matmul`` -- exact-integer
  positional vectors (activation ``[1, 3, 9, 27, 81]`` gives ``byte - 121``;
  tail gives ``byte - 13``), +/-1 data with unit scales (integer results), a
  pure-Python brute force on tiny shapes, and agreement of the three products
  within fp32 rounding of the fp64 one.
* ``get_rows_reference`` -- closed form per element, brute-forced on tiny
  shapes.
* ``compare`` -- adversarial cases from the reference's comparator tests (a
  NaN moved to another position, an infinity with its sign flipped, one bad
  small case hidden next to a huge one).
"""

from __future__ import annotations

import numpy as np

# src/bonsai_tq1/format.py:14-24
BLOCK_SIZE = 128
BLOCK_BYTES = 28
TRIT_BYTES = 26
MAX_FULL_CODE_BYTE = 3**5 - 1
MAX_TAIL_CODE_BYTE = 3**3 - 1
# src/bonsai_tq1/lut23_reorder.py:27-29
M_TILE = 256
CODE_SLOTS = 26
FULL_CODE_SLOTS = 25
TRITS_PER_SLOT = 5
TAIL_FIRST_COLUMN = FULL_CODE_SLOTS * TRITS_PER_SLOT  # src/ternel_mlx/reference.py:38-39
MAX_ORACLE_WEIGHTS = 1 << 27  # src/ternel_mlx/reference.py:43


class OracleFormatError(ValueError):
    """Mirrors ``FormatError(ValueError)`` (src/bonsai_tq1/format.py:33-34)."""


def _as_blocks(blocks) -> np.ndarray:
    """Shape handling of src/bonsai_tq1/format.py:96-102."""
    packed = np.asarray(blocks, dtype=np.uint8)
    if packed.ndim == 1:
        if packed.size % BLOCK_BYTES:
            raise OracleFormatError("TQ1 byte length is not divisible by 28")
        packed = packed.reshape(-1, BLOCK_BYTES)
    if packed.ndim != 2 or packed.shape[1] != BLOCK_BYTES:
        raise OracleFormatError(f"expected TQ1 blocks shaped (N, 28), got {packed.shape}")
    return packed


def count_invalid(blocks) -> tuple[int, int]:
    """Regular bytes > 242 and tail bytes > 26 (src/bonsai_tq1/format.py:104-106)."""
    packed = _as_blocks(blocks)
    payload = packed[:, 2:]
    regular = int(np.count_nonzero(payload[:, :25] > MAX_FULL_CODE_BYTE))
    tail = int(np.count_nonzero(payload[:, 25] > MAX_TAIL_CODE_BYTE))
    return regular, tail


def decode_tq1_blocks(blocks, *, validate: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """``(scales (N,2) u8, codes (N,128) u8)``; src/bonsai_tq1/format.py:94-122.

    Trit ``5j+i`` of a block is ``(byte[2+j] // 3**i) % 3`` for j < 25, and trit
    ``125+i`` is ``(byte[27] // 3**i) % 3``. Fail-closed when ``validate``.
    """
    packed = _as_blocks(blocks)
    if validate:
        regular, tail = count_invalid(packed)
        if regular or tail:
            raise OracleFormatError(f"invalid base-3 bytes: regular={regular}, tail={tail}")
    count = packed.shape[0]
    codes = np.empty((count, BLOCK_SIZE), dtype=np.uint8)
    full = packed[:, 2:27].astype(np.uint16)
    for digit in range(TRITS_PER_SLOT):
        codes[:, digit:TAIL_FIRST_COLUMN:TRITS_PER_SLOT] = ((full // 3**digit) % 3).astype(np.uint8)
    tail = packed[:, 27].astype(np.uint16)
    for digit in range(3):
        codes[:, TAIL_FIRST_COLUMN + digit] = ((tail // 3**digit) % 3).astype(np.uint8)
    return packed[:, :2].copy(), codes


def encode_tq1_blocks(scales, codes) -> np.ndarray:
    """Logical codes 0/1/2 -> 28-byte blocks; src/bonsai_tq1/format.py:66-91."""
    scale_array = np.asarray(scales, dtype=np.uint8).reshape(-1, 2)
    code_array = np.asarray(codes, dtype=np.uint8).reshape(-1, BLOCK_SIZE)
    if scale_array.shape[0] != code_array.shape[0]:
        raise OracleFormatError("scale and code block counts differ")
    invalid = int(np.count_nonzero(code_array > 2))
    if invalid:
        raise OracleFormatError(f"source contains {invalid} non-ternary code(s)")
    count = code_array.shape[0]
    out = np.empty((count, BLOCK_BYTES), dtype=np.uint8)
    out[:, :2] = scale_array
    weights5 = np.array([1, 3, 9, 27, 81], dtype=np.uint16)
    full = code_array[:, :TAIL_FIRST_COLUMN].reshape(count, FULL_CODE_SLOTS, 5).astype(np.uint16)
    out[:, 2:27] = (full * weights5).sum(axis=2).astype(np.uint8)
    out[:, 27] = (code_array[:, TAIL_FIRST_COLUMN:].astype(np.uint16) * weights5[:3]).sum(axis=1).astype(np.uint8)
    return out


SOURCE_BLOCK_BYTES = 34  # src/bonsai_tq1/format.py:15


def decode_q2_blocks(blocks) -> tuple[np.ndarray, np.ndarray]:
    """Prism Q2_0/g128 blocks -> (scale bytes (N, 2), codes (N, 128) in 0..3).

    src/bonsai_tq1/format.py:51-63: code c of a block is bits 2(c % 4) and up of
    quant byte c // 4 (quant bytes follow the two scale bytes).
    """
    source = np.asarray(blocks, dtype=np.uint8)
    if source.ndim == 1:
        source = source.reshape(-1, SOURCE_BLOCK_BYTES)
    quant = source[:, 2:].astype(np.uint8)
    shifts = np.asarray([0, 2, 4, 6], dtype=np.uint8)
    codes = ((quant[:, :, None] >> shifts) & 3).reshape(source.shape[0], BLOCK_SIZE)
    return source[:, :2].copy(), codes.astype(np.uint8)


def q2_dense_weights(blocks, *, rows: int, columns: int) -> np.ndarray:
    """(code - 1) * scale of Q2 blocks in fp64 (src/bonsai_tq1/reference.py:9-52)."""
    scales, codes = decode_q2_blocks(blocks)
    s = scales.reshape(-1).view(np.float16).astype(np.float64)
    return ((codes.astype(np.float64) - 1.0) * s[:, None]).reshape(rows, columns)


def reorder_tensor_arrays(blocks: np.ndarray, *, tile: int) -> tuple[np.ndarray, np.ndarray]:
    """Canonical ``(rows, G, 28)`` -> ``codes[tiles][G][26][tile]``, ``scales[tiles][G][tile][2]``.

    src/bonsai_tq1/lut23_reorder.py:126-142 (last tile zero-padded).
    """
    source = np.asarray(blocks, dtype=np.uint8)
    rows, groups, _ = source.shape
    tiles = -(-rows // tile)
    codes = np.zeros((tiles, groups, CODE_SLOTS, tile), dtype=np.uint8)
    scales = np.zeros((tiles, groups, tile, 2), dtype=np.uint8)
    for index in range(tiles):
        begin = index * tile
        count = min(tile, rows - begin)
        part = source[begin:begin + count]
        codes[index, :, :, :count] = part[:, :, 2:].transpose(1, 2, 0)
        scales[index, :, :count, :] = part[:, :, :2].transpose(1, 0, 2)
    return codes, scales


def restore_tensor_arrays(codes: np.ndarray, scales: np.ndarray, rows: int, *, tile: int) -> np.ndarray:
    """Inverse of :func:`reorder_tensor_arrays`; src/bonsai_tq1/lut23_reorder.py:145-165."""
    groups = codes.shape[1]
    out = np.empty((rows, groups, BLOCK_BYTES), dtype=np.uint8)
    for index in range(codes.shape[0]):
        begin = index * tile
        count = min(tile, rows - begin)
        if count <= 0:
            break
        out[begin:begin + count, :, 2:] = codes[index, :, :, :count].transpose(2, 0, 1)
        out[begin:begin + count, :, :2] = scales[index, :, :count, :].transpose(1, 0, 2)
    return out


def reference_gemv(blocks, activation, *, rows: int, columns: int) -> np.ndarray:
    """Per-row decode-then-dot fp32 GEMV; src/bonsai_tq1/reference.py:14-39,55-65.

    Per row: decode its blocks, ``dot_g = sum_128((t-1) * x, fp32)``, then
    ``sum_g(dot_g * scale_g, fp32)``. Pairwise ``np.sum`` order as the reference.
    """
    if columns % BLOCK_SIZE:
        raise OracleFormatError("columns must be divisible by 128")
    groups = columns // BLOCK_SIZE
    flat = np.asarray(blocks, dtype=np.uint8).reshape(-1)
    if flat.size != rows * groups * BLOCK_BYTES:
        raise OracleFormatError("packed matrix byte count does not match shape")
    x = np.asarray(activation, dtype=np.float32)
    matrix = flat.reshape(rows, groups, BLOCK_BYTES)
    group_x = x.reshape(groups, BLOCK_SIZE)
    out = np.zeros(rows, dtype=np.float32)
    for row in range(rows):
        scale_bits, codes = decode_tq1_blocks(matrix[row])
        weights = codes.astype(np.int8) - 1
        dot = np.sum(weights.astype(np.float32) * group_x, axis=1, dtype=np.float32)
        scale = np.ascontiguousarray(scale_bits).view("<f2").reshape(-1).astype(np.float32)
        out[row] = np.sum(dot * scale, dtype=np.float32)
    return out


def dense_weights(blocks, *, rows: int, columns: int, dtype=np.float64) -> np.ndarray:
    """Dense ``(rows, columns)`` W = (t-1)*scale; src/ternel_mlx/reference.py:155-168.

    Works on canonical blocks (the build's device layout) instead of the tiled
    pair; the reference first restores canonical blocks with ``unpack_blocks``.
    """
    if rows * columns > MAX_ORACLE_WEIGHTS:
        raise OracleFormatError(
            f"refusing to densify {rows}x{columns} weights; the oracle is capped at "
            f"{MAX_ORACLE_WEIGHTS} elements"
        )
    flat = np.asarray(blocks, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    scale_bits, trits = decode_tq1_blocks(flat, validate=True)
    dt = np.dtype(dtype)
    weights = trits.astype(np.int8).astype(dt) - dt.type(1)
    scale = np.ascontiguousarray(scale_bits).view("<f2").astype(dt).reshape(-1, 1)
    with np.errstate(invalid="ignore", over="ignore"):
        return (weights * scale).reshape(rows, columns)


def oracle_matmul(blocks, x, *, rows: int, columns: int) -> np.ndarray:
    """fp64 dense product, the exactness oracle; src/ternel_mlx/reference.py:171-177."""
    activation = np.asarray(x, dtype=np.float64)
    if activation.ndim != 2 or activation.shape[1] != columns:
        raise OracleFormatError(f"activations must be (batch, {columns}), got shape {activation.shape}")
    weights = dense_weights(blocks, rows=rows, columns=columns, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        return activation @ weights.T


def _digit_table(entries: int, digits: int) -> np.ndarray:
    index = np.arange(entries, dtype=np.int64)
    return np.stack([(index // 3**d) % 3 for d in range(digits)]).astype(np.float32) - 1.0


def build_group_tables(activations: np.ndarray):
    """LUT23 tables for one group, fp32; src/ternel_mlx/reference.py:56-86.

    ``L2[s][c] = (c%3-1)x0 + (c/3-1)x1``; ``L3[s][c] = (c%3-1)x2 + ((c/3)%3-1)x3 + (c/9-1)x4``;
    ``tail[c]`` over x125..127, each evaluated left to right in fp32.
    """
    x = np.asarray(activations, dtype=np.float32)
    slots = x[:TAIL_FIRST_COLUMN].reshape(FULL_CODE_SLOTS, TRITS_PER_SLOT)
    d2 = _digit_table(9, 2)
    d3 = _digit_table(27, 3)
    with np.errstate(invalid="ignore", over="ignore"):
        l2 = (slots[:, 0:1] * d2[0] + slots[:, 1:2] * d2[1]).astype(np.float32)
        l3 = (slots[:, 2:3] * d3[0] + slots[:, 3:4] * d3[1] + slots[:, 4:5] * d3[2]).astype(np.float32)
        t = x[TAIL_FIRST_COLUMN:]
        tail = (t[0] * d3[0] + t[1] * d3[1] + t[2] * d3[2]).astype(np.float32)
    return l2, l3, tail


def _fma32(a, b, c):
    """Correctly rounded fp32 fma via fp64; src/ternel_mlx/reference.py:89-98."""
    with np.errstate(invalid="ignore", over="ignore"):
        return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def lut23_matmul(blocks, x, *, rows: int, columns: int) -> np.ndarray:
    """Table-driven product in the LUT23 kernel's summation order.

    src/ternel_mlx/reference.py:117-152 (the Metal kernel order of
    src/ternel_mlx/kernels.py:279-324): per group ``sum = 0; for s in 0..24:
    sum += (L2[s][lo] + L3[s][hi]); sum += tail[b25]; acc = fma(scale, sum, acc)``
    with ``hi = (p*57)>>9``, ``lo = p - 9*hi``.
    """
    activation = np.asarray(x, dtype=np.float32)
    groups = columns // BLOCK_SIZE
    matrix = np.asarray(blocks, dtype=np.uint8).reshape(rows, groups, BLOCK_BYTES)
    full = matrix[:, :, 2:27].astype(np.uint32)
    high = (full * np.uint32(57)) >> np.uint32(9)
    low = full - np.uint32(9) * high
    tail_codes = matrix[:, :, 27]
    scale = np.ascontiguousarray(matrix[:, :, :2]).view("<f2").reshape(rows, groups).astype(np.float32)
    out = np.zeros((activation.shape[0], rows), dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for sample in range(activation.shape[0]):
            acc = np.zeros(rows, dtype=np.float32)
            for g in range(groups):
                l2, l3, tail = build_group_tables(activation[sample, g * BLOCK_SIZE:(g + 1) * BLOCK_SIZE])
                total = np.zeros(rows, dtype=np.float32)
                for s in range(FULL_CODE_SLOTS):
                    total += l2[s][low[:, g, s]] + l3[s][high[:, g, s]]
                total += tail[tail_codes[:, g]]
                acc = _fma32(scale[:, g], total, acc)
            out[sample] = acc
    return out


def get_rows_reference(blocks, indices, *, rows: int, columns: int, dtype=np.float32,
                       out_of_range: str = "zero") -> np.ndarray:
    """Decode only the requested rows; src/ternel_mlx/reference.py:196-230.

    ``out[t, c] = (trit(row, c) - 1) * scale``. The CPU reference rejects ids
    outside ``[0, rows)``; the Metal kernel writes zeros for them
    (src/ternel_mlx/kernels.py:869-880). ``out_of_range`` picks which.
    """
    ids = np.asarray(indices).reshape(-1).astype(np.int64)
    bad = (ids < 0) | (ids >= rows)
    if out_of_range == "raise" and bad.any():
        raise OracleFormatError(f"indices fall outside [0, {rows})")
    groups = columns // BLOCK_SIZE
    matrix = np.asarray(blocks, dtype=np.uint8).reshape(rows, groups, BLOCK_BYTES)
    safe = np.where(bad, 0, ids)
    selected = matrix[safe].reshape(-1, BLOCK_BYTES)
    scale_bits, trits = decode_tq1_blocks(selected, validate=False)
    dt = np.dtype(dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        weights = trits.astype(np.int8).astype(dt) - dt.type(1)
        scale = np.ascontiguousarray(scale_bits).view("<f2").astype(dt).reshape(-1, 1)
        out = (weights * scale).reshape(ids.size, columns)
    out[bad] = 0
    return out


def _classify(values: np.ndarray) -> np.ndarray:
    """Finite / +inf / -inf / NaN per element; src/ternel_mlx/kernel_gate.py:275-287."""
    classes = np.zeros(values.shape, dtype=np.int8)
    classes[np.isposinf(values)] = 1
    classes[np.isneginf(values)] = 2
    classes[np.isnan(values)] = 3
    return classes


def compare(candidate, reference) -> dict:
    """Per-case normalised error + non-finite pattern; src/ternel_mlx/kernel_gate.py:290-372.

    Both sides are ``(case, output)``. Returns ``normalised_max_abs_error`` (max
    over cases of max|got-want| / max|want| in that case, finite entries only),
    ``pattern_mismatches`` (positions whose finite/+inf/-inf/NaN class differs),
    and ``bit_exact``.
    """
    got = np.asarray(candidate, dtype=np.float64)
    want = np.asarray(reference, dtype=np.float64)
    if got.shape != want.shape or got.ndim != 2:
        raise OracleFormatError(f"cannot compare {got.shape} against {want.shape}")
    pattern = int(np.count_nonzero(_classify(got) != _classify(want)))
    finite = np.isfinite(got) & np.isfinite(want)
    a = np.where(finite, got, 0.0)
    b = np.where(finite, want, 0.0)
    error = np.abs(a - b)
    magnitude = np.abs(b).max(axis=1)
    scale = np.where(magnitude > 0.0, magnitude, 1.0)
    normalised = error / scale[:, None]
    return {
        "normalised_max_abs_error": float(normalised.max()) if normalised.size else 0.0,
        "worst_case": int(np.argmax(normalised.max(axis=1))) if normalised.size else 0,
        "pattern_mismatches": pattern,
        "bit_exact": bool(error.max() == 0.0 and pattern == 0) if error.size else pattern == 0,
    }


def cpu_decode(blocks, *, rows: int, columns: int) -> np.ndarray:
    """The BASELINE CPU arm's decode: whole-matrix decode -> dense fp32 W = (t-1)*scale.

    Restates the reference's Python decoder (src/bonsai_tq1/format.py:94-122,
    validating) and densification (src/ternel_mlx/reference.py:155-168) in fp32.
    Timed by ``bench.py`` as part of the reported CPU baseline; never used by the product.
    """
    flat = np.asarray(blocks, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    scale_bits, trits = decode_tq1_blocks(flat, validate=True)
    weights = trits.astype(np.float32) - np.float32(1.0)
    weights *= np.ascontiguousarray(scale_bits).view("<f2").astype(np.float32).reshape(-1, 1)
    return weights.reshape(rows, columns)


def cpu_matmul(dense: np.ndarray, x) -> np.ndarray:
    """The BASELINE CPU arm's product: ``x @ W.T`` in fp32 (numpy BLAS) -> fp16;
    src/ternel_mlx/reference.py:171-177 at the reference's fp32 CPU precision."""
    return (np.asarray(x, dtype=np.float32) @ dense.T).astype(np.float16)


def cpu_decode_matmul(blocks, x, *, rows: int, columns: int) -> np.ndarray:
    """The BASELINE CPU arm end to end: ``cpu_decode`` then ``cpu_matmul``."""
    return cpu_matmul(cpu_decode(blocks, rows=rows, columns=columns), x)
