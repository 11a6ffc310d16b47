"""TQ1_G128 block format: constants, the error type, the host encoder and the
device-side decode/validation entry points.

Mirrors the public surface of ``bonsai_tq1.format`` (src/bonsai_tq1/format.py):
same constants, ``FormatError(ValueError)``, ``encode_tq1_blocks`` and
``decode_tq1_blocks`` with the same shapes and error messages. Decoding and
validation run on the GPU through the C ABI; encoding is host-side data
preparation (the reference's conversion is offline numpy as well).
"""

from __future__ import annotations

import numpy as np
import torch

BLOCK_SIZE = 128
BLOCK_BYTES = 28
TRIT_BYTES = 26
CODE_SLOTS = 26
FULL_CODE_SLOTS = 25
MAX_FULL_CODE_BYTE = 3**5 - 1
MAX_TAIL_CODE_BYTE = 3**3 - 1
POWERS5 = np.asarray([1, 3, 9, 27, 81], dtype=np.uint16)
POWERS3 = np.asarray([1, 3, 9], dtype=np.uint16)


class FormatError(ValueError):
    """Malformed packed data or geometry (src/bonsai_tq1/format.py:33-34)."""


def encode_tq1_blocks(scales, codes) -> np.ndarray:
    """Encode logical codes 0/1/2 as 28-byte blocks (src/bonsai_tq1/format.py:66-91).

    ``scales``: (N, 2) raw fp16 scale bytes; ``codes``: (N, 128) values in {0,1,2}.
    Byte ``2+j`` = sum_i codes[5j+i] * 3**i, byte 27 = sum_i codes[125+i] * 3**i.
    """
    scale_array = np.asarray(scales, dtype=np.uint8)
    code_array = np.asarray(codes, dtype=np.uint8)
    if scale_array.ndim == 1:
        scale_array = scale_array.reshape(-1, 2)
    if code_array.ndim == 1:
        code_array = code_array.reshape(-1, BLOCK_SIZE)
    if scale_array.ndim != 2 or scale_array.shape[1] != 2:
        raise FormatError(f"expected scale bytes shaped (N, 2), got {scale_array.shape}")
    if code_array.ndim != 2 or code_array.shape[1] != BLOCK_SIZE:
        raise FormatError(f"expected codes shaped (N, 128), got {code_array.shape}")
    if scale_array.shape[0] != code_array.shape[0]:
        raise FormatError("scale and code block counts differ")
    invalid = int(np.count_nonzero(code_array > 2))
    if invalid:
        raise FormatError(f"source contains {invalid} non-ternary code(s)")
    count = code_array.shape[0]
    result = np.empty((count, BLOCK_BYTES), dtype=np.uint8)
    result[:, :2] = scale_array
    slots = code_array[:, :125].reshape(count, FULL_CODE_SLOTS, 5).astype(np.uint16)
    result[:, 2:27] = (slots * POWERS5).sum(axis=2, dtype=np.uint16).astype(np.uint8)
    result[:, 27] = (code_array[:, 125:].astype(np.uint16) * POWERS3).sum(axis=1, dtype=np.uint16).astype(np.uint8)
    return result


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("the TQ1 engine needs a ROCm GPU (torch.cuda is unavailable)")
    return torch.device("cuda", torch.cuda.current_device())


def as_device_blocks(blocks) -> torch.Tensor:
    """Canonical blocks as a contiguous uint8 device tensor of shape (N, 28)."""
    if isinstance(blocks, torch.Tensor):
        tensor = blocks
    else:
        tensor = torch.from_numpy(np.ascontiguousarray(np.asarray(blocks, dtype=np.uint8)))
    if tensor.dtype != torch.uint8:
        raise FormatError(f"canonical blocks must be uint8, got {tensor.dtype}")
    if tensor.ndim == 1:
        if tensor.numel() % BLOCK_BYTES:
            raise FormatError("TQ1 byte length is not divisible by 28")
        tensor = tensor.reshape(-1, BLOCK_BYTES)
    elif tensor.ndim >= 2 and tensor.shape[-1] == BLOCK_BYTES:
        tensor = tensor.reshape(-1, BLOCK_BYTES)
    if tensor.ndim != 2 or tensor.shape[1] != BLOCK_BYTES:
        raise FormatError(f"expected TQ1 blocks shaped (N, 28), got {tuple(tensor.shape)}")
    if not tensor.is_cuda:
        tensor = tensor.to(_device())
    return tensor.contiguous()


def count_invalid_bytes(blocks) -> tuple[int, int]:
    """(regular bytes > 242, tail bytes > 26), counted on the GPU."""
    from . import _lib

    device_blocks = as_device_blocks(blocks)
    counters = torch.empty(2, dtype=torch.int64, device=device_blocks.device)
    stream = torch.cuda.current_stream(device_blocks.device).cuda_stream
    _lib.check(
        _lib.lib().ternel_tq1_validate(
            device_blocks.data_ptr(), device_blocks.shape[0], counters.data_ptr(), stream
        )
    )
    regular, tail = (int(v) for v in counters.cpu().tolist())
    return regular, tail


def validate_blocks(blocks) -> None:
    """Raise the reference's FormatError if any code byte is out of range.

    Message of src/bonsai_tq1/format.py:104-110.
    """
    regular, tail = count_invalid_bytes(blocks)
    if regular or tail:
        raise FormatError(f"invalid base-3 bytes: regular={regular}, tail={tail}")


def validate_packed_codes(blocks) -> None:
    """Load-time full scan with the message of src/ternel_mlx/packing.py:29-48."""
    regular, tail = count_invalid_bytes(blocks)
    if regular or tail:
        raise FormatError(
            f"packed codes contain out-of-range base-3 bytes: regular={regular} "
            f"(max {MAX_FULL_CODE_BYTE}), tail={tail} (max {MAX_TAIL_CODE_BYTE})"
        )


SOURCE_BLOCK_BYTES = 34  # Prism Q2_0/g128: fp16 scale + 32 bytes of 2-bit codes


def convert_q2_blocks(blocks):
    """Q2_0/g128 source blocks -> canonical TQ1_G128 blocks on the GPU.

    ``decode_q2_blocks`` + ``encode_tq1_blocks`` of src/bonsai_tq1/format.py
    :51-91 in one device pass, with their shape checks and messages; a code of
    3 (no ternary meaning) rejects the whole source. Returns numpy blocks for
    numpy input and device blocks for tensor input, shaped (N, 28).
    """
    from . import _lib

    if isinstance(blocks, torch.Tensor):
        source = blocks
    else:
        source = torch.from_numpy(np.ascontiguousarray(np.asarray(blocks, dtype=np.uint8)))
    if source.dtype != torch.uint8:
        raise FormatError(f"Q2 blocks must be uint8, got {source.dtype}")
    if source.ndim == 1:
        if source.numel() % SOURCE_BLOCK_BYTES:
            raise FormatError("Q2 byte length is not divisible by 34")
        source = source.reshape(-1, SOURCE_BLOCK_BYTES)
    if source.ndim != 2 or source.shape[1] != SOURCE_BLOCK_BYTES:
        raise FormatError(f"expected Q2 blocks shaped (N, 34), got {tuple(source.shape)}")
    device_source = (source if source.is_cuda else source.to(_device())).contiguous()
    out = torch.empty((device_source.shape[0], BLOCK_BYTES), dtype=torch.uint8, device=device_source.device)
    bad = torch.empty(1, dtype=torch.int64, device=device_source.device)
    stream = torch.cuda.current_stream(device_source.device).cuda_stream
    _lib.check(_lib.lib().ternel_tq1_from_q2(device_source.data_ptr(), device_source.shape[0], out.data_ptr(),
                                             bad.data_ptr(), stream))
    invalid = int(bad.item())
    if invalid:
        raise FormatError(f"source contains {invalid} non-ternary code(s)")
    return out if isinstance(blocks, torch.Tensor) else out.cpu().numpy()


def decode_tq1_blocks(blocks, *, validate: bool = True):
    """Decode 28-byte blocks to ``(scales (N,2) u8, codes (N,128) u8)`` on the GPU.

    Same contract as src/bonsai_tq1/format.py:94-122: fail-closed when
    ``validate``; with ``validate=False`` every byte is decoded as
    ``(b // 3**i) % 3``. Returns numpy arrays for numpy input and device tensors
    for tensor input.
    """
    from . import _lib

    numpy_in = not isinstance(blocks, torch.Tensor)
    device_blocks = as_device_blocks(blocks)
    if validate:
        validate_blocks(device_blocks)
    count = device_blocks.shape[0]
    scales = torch.empty((count, 2), dtype=torch.uint8, device=device_blocks.device)
    codes = torch.empty((count, BLOCK_SIZE), dtype=torch.uint8, device=device_blocks.device)
    stream = torch.cuda.current_stream(device_blocks.device).cuda_stream
    _lib.check(
        _lib.lib().ternel_tq1_decode(
            device_blocks.data_ptr(), count, scales.data_ptr(), codes.data_ptr(), stream
        )
    )
    if numpy_in:
        return scales.cpu().numpy(), codes.cpu().numpy()
    return scales, codes
