"""Synthetic TQ1_G128 weights and activations with the benchmark distributions.

Trits are i.i.d. with P(t=0, 1, 2) = (0.3, 0.4, 0.3), i.e. weights -1/0/+1 with
P(0) = 0.4; scales are fp16(|N(0, 0.02)| + 1e-4); activations fp16 N(0, sigma).
``host_*`` build small tensors with numpy (seeded ``default_rng``); ``device_*``
build large ones directly on the GPU with torch in chunks, so a multi-GB weight
stream never passes through host memory.
"""

from __future__ import annotations

import numpy as np
import torch

from .format import BLOCK_BYTES, BLOCK_SIZE, encode_tq1_blocks

TRIT_PROBABILITIES = (0.3, 0.4, 0.3)
SCALE_SIGMA = 0.02
SCALE_FLOOR = 1e-4
SEED_BASE = 20261201


def host_trits(rng: np.random.Generator, count: int) -> np.ndarray:
    return rng.choice(3, size=(count, BLOCK_SIZE), p=TRIT_PROBABILITIES).astype(np.uint8)


def host_scale_bits(rng: np.random.Generator, count: int) -> np.ndarray:
    scales = (np.abs(rng.normal(0.0, SCALE_SIGMA, size=count)) + SCALE_FLOOR).astype(np.float16)
    return scales.view(np.uint8).reshape(count, 2)


def host_blocks(rows: int, columns: int, *, seed: int) -> np.ndarray:
    """Canonical ``(rows, columns/128, 28)`` blocks, numpy."""
    rng = np.random.default_rng(seed)
    groups = rows * (columns // BLOCK_SIZE)
    blocks = encode_tq1_blocks(host_scale_bits(rng, groups), host_trits(rng, groups))
    return blocks.reshape(rows, columns // BLOCK_SIZE, BLOCK_BYTES)


def host_activations(batch: int, columns: int, *, seed: int, sigma: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.normal(0.0, sigma, size=(batch, columns)).astype(np.float16)


def _device_trit_bytes(count: int, digits: int, gen: torch.Generator, device) -> torch.Tensor:
    u = torch.rand((count, digits), generator=gen, device=device)
    t = (u >= TRIT_PROBABILITIES[0]).to(torch.int32) + (u >= TRIT_PROBABILITIES[0] + TRIT_PROBABILITIES[1]).to(torch.int32)
    powers = torch.tensor([1, 3, 9, 27, 81][:digits], dtype=torch.int32, device=device)
    return (t * powers).sum(dim=1).to(torch.uint8)


def device_blocks(rows: int, columns: int, *, seed: int, device=None, chunk_blocks: int = 1 << 20) -> torch.Tensor:
    """Canonical blocks generated on the GPU: ``(rows, columns/128, 28)`` uint8."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    groups = rows * (columns // BLOCK_SIZE)
    out = torch.empty((groups, BLOCK_BYTES), dtype=torch.uint8, device=device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for start in range(0, groups, chunk_blocks):
        n = min(chunk_blocks, groups - start)
        scales = (torch.randn(n, generator=gen, device=device) * SCALE_SIGMA).abs_() + SCALE_FLOOR
        out[start:start + n, 0:2] = scales.to(torch.float16).view(torch.uint8).reshape(n, 2)
        out[start:start + n, 2:27] = _device_trit_bytes(n * 25, 5, gen, device).reshape(n, 25)
        out[start:start + n, 27] = _device_trit_bytes(n, 3, gen, device)
    return out.reshape(rows, columns // BLOCK_SIZE, BLOCK_BYTES)


def device_activations(batch: int, columns: int, *, seed: int, sigma: float = 1.0, device=None) -> torch.Tensor:
    device = device or torch.device("cuda", torch.cuda.current_device())
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return (torch.randn((batch, columns), generator=gen, device=device) * sigma).to(torch.float16)
