"""torch modules that execute packed TQ1_G128 weights without unpacking them.

Twins of the reference's module API (src/ternel_mlx/modules.py:425-549):
``packed_matmul(codes, scales, x, *, layout)``, ``PackedLinear`` and
``PackedEmbedding`` keep their names, constructor arguments, call signatures,
output shapes/dtypes and FormatError messages, and their state is the
reference's: ``codes`` (uint8 ``(tiles, G, 26, tile)``) and ``scales`` (uint16
raw fp16 bits ``(tiles, G, tile)``) -- the state-dict keys the MLX artifact
uses (src/ternel_mlx/layout.py:37-38), loadable with ``load_state_dict`` or
``load_weights([("codes", c), ("scales", s)])``.

What the modules keep in device memory is one copy of the weight, as the
engine's packed words (the same 28 bytes per 128 weights, permuted at 4-byte
granularity for the gfx950 kernels). ``codes`` and ``scales`` read back as
device tensors, derived from the words once per weight version on the GPU;
assigning either converts on the GPU (with the fail-closed byte scan).

``replace_with_packed`` is the torch counterpart of
src/ternel_mlx/packed_model.py:72-92: it swaps every bias-free ``nn.Linear`` and
every ``nn.Embedding`` of a model for the packed twins.
"""

from __future__ import annotations

import weakref

import numpy as np
import torch
from torch import nn

from .format import BLOCK_BYTES, FormatError, as_device_blocks, validate_packed_codes
from .kernels import (
    GemmConfig,
    MatmulConfig,
    pack_weights,
    packed_shape,
    tiled_from_words,
    tq1_gemm_words,
    tq1_get_rows_canonical,
    tq1_get_rows_words,
    tq1_matmul_words,
    tq1_swiglu_words,
    unpack_weights,
    words_from_tiled,
    words_of,
)
from .layout import PackedTensorLayout, interleave_gate_up, unpack_blocks

# Dispatch (src/ternel_mlx/modules.py:331-422, re-measured for MI355X): the
# LUT23 kernels for small batches, the MFMA kernels above them. The LUT kernel's
# cost grows linearly with the batch (one table set per vector) while its bytes
# do not, so it only pays while the weight stream dominates. The rule lives in
# the library (ternel_tq1_linear_kernel, replayed against a measured sweep in
# tests/test_dispatch.py); LUT23_MAX_BATCH is its bound for matrices of 16 MiB
# of packed weights or more, the 27B MLP shapes (smaller matrices: 4 rows).
LUT23_MAX_BATCH = 3
_KERNEL_NAMES = {100: "lut23", 1: "gemm", 2: "gemm", 3: "gemm"}


def select_kernel(layout: PackedTensorLayout, batch: int, dtype: torch.dtype) -> str:
    """``"lut23"`` or ``"gemm"`` for ``batch`` activation rows: the library's own choice."""
    from . import _lib
    from .kernels import _DTYPE_CODE

    code = _lib.lib().ternel_tq1_linear_kernel(batch, layout.rows, layout.columns, _DTYPE_CODE[dtype])
    if code < 0:
        raise FormatError(_lib.lib().ternel_tq1_last_error().decode())
    return _KERNEL_NAMES[code]


def matmul_words(packed: torch.Tensor, x: torch.Tensor, *, layout: PackedTensorLayout) -> torch.Tensor:
    """``x @ W.T`` for packed words ``W``, choosing the kernel by activation rows
    and keeping the leading dimensions of ``x``."""
    if x.shape[-1] != layout.columns:
        raise FormatError(f"activation has {x.shape[-1]} columns, weight expects {layout.columns}")
    flat = x.reshape(-1, layout.columns)
    if select_kernel(layout, flat.shape[0], flat.dtype) == "gemm":
        out = tq1_gemm_words(packed, flat, layout=layout, config=GemmConfig())
    else:
        out = tq1_matmul_words(packed, flat, layout=layout, config=MatmulConfig())
    return out.reshape(*x.shape[:-1], layout.rows)


def packed_matmul(codes: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, *,
                  layout: PackedTensorLayout) -> torch.Tensor:
    """``x @ W.T`` for a packed ``W`` given as the reference's tiled pair,
    choosing the kernel by activation rows (src/ternel_mlx/modules.py:425-457).
    The pair is converted to packed words once and cached while it lives
    unchanged (``kernels.words_of``)."""
    if x.shape[-1] != layout.columns:
        raise FormatError(f"activation has {x.shape[-1]} columns, weight expects {layout.columns}")
    packed, pair_layout = words_of(codes, scales, groups_per_row=layout.groups_per_row, tile=layout.tile)
    if (pair_layout.rows, pair_layout.columns) != (layout.rows, layout.columns):
        raise FormatError(f"codes/scales hold a {pair_layout.rows}x{pair_layout.columns} tensor, "
                          f"the layout {layout.rows}x{layout.columns}")
    return matmul_words(packed, x, layout=layout)


class _PackedWeight(nn.Module):
    """Storage and loading of one packed weight: the packed words in device
    memory, the reference's ``codes``/``scales`` as the state."""

    def __init__(self, layout: PackedTensorLayout, device=None) -> None:
        super().__init__()
        self.layout = layout
        if device is None and torch.cuda.is_available():
            device = torch.device("cuda", torch.cuda.current_device())
        # The words are derived state: the state dict holds codes and scales.
        self.register_buffer("packed", torch.zeros(packed_shape(layout), dtype=torch.int32, device=device),
                             persistent=False)

    # -- loading --------------------------------------------------------------
    def load_blocks(self, blocks, *, validate: bool = True) -> None:
        """Load canonical blocks (any shape holding ``rows * G`` 28-byte blocks).

        Every byte is scanned on the GPU first (fail-closed), then the blocks are
        permuted into the packed words.
        """
        tensor = as_device_blocks(blocks)
        if tensor.shape[0] != self.layout.groups:
            raise FormatError(
                f"expected {self.layout.groups} blocks for {self.layout.rows}x{self.layout.columns}, "
                f"got {tensor.shape[0]}"
            )
        if validate:
            validate_packed_codes(tensor)
        self.packed = pack_weights(tensor, layout=self.layout)

    def load_packed(self, codes, scales, *, validate: bool = True) -> None:
        """Load the reference's tiled ``codes`` (u8) / ``scales`` (<u2) arrays:
        device tensors are converted on the GPU, host arrays uploaded first."""
        device = self.packed.device if self.packed.is_cuda else torch.device("cuda", torch.cuda.current_device())
        codes_t = _as_device(codes, torch.uint8, device)
        scales_t = _as_device(scales, torch.uint16, device)
        self.packed = words_from_tiled(codes_t, scales_t, layout=self.layout, validate=validate)

    def load_weights(self, weights, strict: bool = True) -> "_PackedWeight":
        """MLX-style ``load_weights([("codes", c), ("scales", s)])`` (tests/test_mlx_modules.py:132-133)."""
        named = dict(weights)
        if "blocks" in named:
            self.load_blocks(named.pop("blocks"))
        elif "codes" in named or "scales" in named:
            if "codes" not in named or "scales" not in named:
                raise FormatError("codes and scales must be loaded together")
            self.load_packed(named.pop("codes"), named.pop("scales"))
        if strict and named:
            raise FormatError(f"unexpected weights: {sorted(named)}")
        return self

    def load_sidecar(self, path, name: str, *, validate: bool = True) -> "_PackedWeight":
        """Load tensor ``name`` of a canonical sidecar (src/bonsai_tq1/format.py:150-246)."""
        from .artifact import load_sidecar_tensor

        layout, packed = load_sidecar_tensor(path, name, device=self.packed.device, validate=validate)
        self._take(layout, packed)
        return self

    def load_safetensors(self, path, name: str, *, validate: bool = True) -> "_PackedWeight":
        """Load ``<name>.codes`` / ``<name>.scales`` of an MLX artifact (src/ternel_mlx/layout.py:37-38)."""
        from .artifact import load_safetensors_tensor

        layout, packed = load_safetensors_tensor(path, name, device=self.packed.device, validate=validate)
        self._take(layout, packed)
        return self

    def _take(self, layout: PackedTensorLayout, packed: torch.Tensor) -> None:
        if (layout.rows, layout.columns) != (self.layout.rows, self.layout.columns):
            raise FormatError(f"artifact tensor is {layout.rows}x{layout.columns}, the module "
                              f"{self.layout.rows}x{self.layout.columns}")
        self.packed = packed

    # -- the reference's state ------------------------------------------------
    def _tiled_pair(self) -> tuple[torch.Tensor, torch.Tensor]:
        # Derived on every access and not kept: the module holds one copy of
        # the weight (the words), as the reference holds one (its codes and
        # scales, src/ternel_mlx/modules.py:472-473,516-517). The state dict
        # takes both arrays from one conversion.
        return tiled_from_words(self.packed, layout=self.layout)

    @property
    def blocks(self) -> torch.Tensor:
        """Canonical ``(rows, G, 28)`` device blocks, by exact inverse permutation."""
        return unpack_weights(self.packed, layout=self.layout)

    @property
    def codes(self) -> torch.Tensor:
        """The reference's tiled code array (uint8, device), by exact permutation."""
        return self._tiled_pair()[0]

    @codes.setter
    def codes(self, value) -> None:
        self.load_packed(value, self.scales)

    @property
    def scales(self) -> torch.Tensor:
        """The reference's tiled scale array (uint16 raw fp16 bits, device)."""
        return self._tiled_pair()[1]

    @scales.setter
    def scales(self, value) -> None:
        self.load_packed(self.codes, value)

    def _save_to_state_dict(self, destination, prefix, keep_vars) -> None:
        super()._save_to_state_dict(destination, prefix, keep_vars)
        codes, scales = self._tiled_pair()
        destination[prefix + "codes"] = codes if keep_vars else codes.detach()
        destination[prefix + "scales"] = scales if keep_vars else scales.detach()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs) -> None:
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)
        keys = (prefix + "codes", prefix + "scales")
        # Not registered parameters or buffers: the base class counts them as unexpected.
        for k in keys:
            if k in unexpected_keys:
                unexpected_keys.remove(k)
        present = [k in state_dict for k in keys]
        if all(present):
            try:
                self.load_packed(state_dict[keys[0]], state_dict[keys[1]])
            except FormatError as exc:
                error_msgs.append(f"{prefix}codes/scales: {exc}")
        else:
            missing_keys.extend(k for k, p in zip(keys, present) if not p)


def _as_device(array, dtype: torch.dtype, device) -> torch.Tensor:
    if isinstance(array, torch.Tensor):
        tensor = array
        if dtype == torch.uint16 and tensor.dtype == torch.int16:
            tensor = tensor.view(torch.uint16)
    else:
        host = np.ascontiguousarray(array)
        if dtype == torch.uint16:
            host = host.view("<u2") if host.dtype.itemsize == 2 else host.astype("<u2")
            tensor = torch.from_numpy(host.view(np.int16)).view(torch.uint16)
        else:
            tensor = torch.from_numpy(host)
    if tensor.dtype != dtype:
        raise FormatError(f"expected {dtype}, got {tensor.dtype}")
    return tensor.to(device).contiguous()


class PackedLinear(_PackedWeight):
    """Bias-free linear layer whose weight stays in TQ1_G128 (src/ternel_mlx/modules.py:460-495)."""

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "PackedLinear":
        if linear.bias is not None:
            raise FormatError("a packed linear layer cannot carry a bias")
        rows, columns = linear.weight.shape
        return cls(PackedTensorLayout.for_tensor(rows, columns), device=linear.weight.device)

    @classmethod
    def from_sidecar(cls, path, name: str, *, device=None) -> "PackedLinear":
        """The sidecar tensor ``name`` as a layer (shape from its manifest entry)."""
        from .artifact import read_sidecar, sidecar_tensors

        entry = sidecar_tensors(read_sidecar(path)[1]).get(name)
        if entry is None:
            raise FormatError(f"sidecar has no tensor {name!r}")
        return cls(entry.layout, device=device).load_sidecar(path, name)

    @classmethod
    def from_safetensors(cls, path, name: str, *, device=None) -> "PackedLinear":
        """The MLX-artifact tensor ``name`` as a layer (shape from its tiled arrays)."""
        from .artifact import load_safetensors_tensor

        layout, packed = load_safetensors_tensor(path, name, device=device)
        layer = cls(layout, device=packed.device)
        layer.packed = packed
        return layer

    def extra_repr(self) -> str:
        return (f"{self.layout.columns} -> {self.layout.rows}, tile={self.layout.tile}, "
                f"{self.layout.bits_per_weight:.3f} bits/weight")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return matmul_words(self.packed, x, layout=self.layout)


class PackedEmbedding(_PackedWeight):
    """Token embedding decoded one row at a time (src/ternel_mlx/modules.py:498-549)."""

    def __init__(self, layout: PackedTensorLayout, *, dtype: torch.dtype, device=None,
                 canonical_rows: bool = False) -> None:
        super().__init__(layout, device=device)
        self.dtype = dtype
        # Opt-in second copy of the table as canonical row-major blocks, which
        # a gather reads contiguously (an 8192-token prefill gather ~2.6x
        # faster) at the cost of the table's size again in device memory
        # (170 MB at 151,936 x 5120). Off by default: one copy, as the
        # reference keeps.
        self.canonical_rows = canonical_rows

    @classmethod
    def from_embedding(cls, embedding: nn.Embedding, *, dtype: torch.dtype) -> "PackedEmbedding":
        rows, columns = embedding.weight.shape
        return cls(PackedTensorLayout.for_tensor(rows, columns), dtype=dtype, device=embedding.weight.device)

    @classmethod
    def from_sidecar(cls, path, name: str, *, dtype: torch.dtype, device=None) -> "PackedEmbedding":
        from .artifact import read_sidecar, sidecar_tensors

        entry = sidecar_tensors(read_sidecar(path)[1]).get(name)
        if entry is None:
            raise FormatError(f"sidecar has no tensor {name!r}")
        return cls(entry.layout, dtype=dtype, device=device).load_sidecar(path, name)

    @classmethod
    def from_safetensors(cls, path, name: str, *, dtype: torch.dtype, device=None) -> "PackedEmbedding":
        from .artifact import load_safetensors_tensor

        layout, packed = load_safetensors_tensor(path, name, device=device)
        table = cls(layout, dtype=dtype, device=packed.device)
        table.packed = packed
        return table

    def extra_repr(self) -> str:
        return f"{self.layout.rows} x {self.layout.columns}, tile={self.layout.tile}, {self.dtype}"

    def forward(self, indices: torch.Tensor) -> torch.Tensor:
        """Rows for ``indices`` of any shape and integer dtype; ids outside the
        table read as zeros (src/ternel_mlx/modules.py:527-545)."""
        flat = indices.reshape(-1)
        if self.canonical_rows:
            rows = tq1_get_rows_canonical(self.row_blocks(), flat, layout=self.layout, dtype=self.dtype)
        else:
            rows = tq1_get_rows_words(self.packed, flat, layout=self.layout, dtype=self.dtype)
        return rows.reshape(*indices.shape, self.layout.columns)

    def row_blocks(self) -> torch.Tensor:
        """The table as canonical ``(rows, G, 28)`` device blocks (``canonical_rows``),
        derived from the packed words on first use and again whenever they are
        replaced or written. Not part of the state dict. Call it once before
        capturing a graph that gathers, so the capture holds no rebuild."""
        # Keyed on the words tensor itself (a weak reference, so a replaced
        # tensor whose storage the allocator hands to the next load can never
        # match) and its version counter (in-place writes).
        source = getattr(self, "_row_blocks_source", None)
        if source is None or source() is not self.packed or self._row_blocks_version != self.packed._version:
            self._row_blocks = unpack_weights(self.packed, layout=self.layout)
            self._row_blocks_source = weakref.ref(self.packed)
            self._row_blocks_version = self.packed._version
        return self._row_blocks

    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        """Tied output head: the embedding table used as a matmul."""
        return matmul_words(self.packed, x, layout=self.layout)


class PackedSwiGLU(nn.Module):
    """The gate and up projections of a SwiGLU MLP as one packed weight, with
    the elementwise step fused: ``forward(x) = SiLU(x @ gate.T) * (x @ up.T)``,
    each projection rounded to ``x.dtype`` as the unfused layers would return
    it. The weight's rows alternate gate, up (``layout.interleave_gate_up``);
    one launch reads both projections' 28-byte blocks and writes ``hidden``
    values per vector. No counterpart module in the reference (its MLP runs the
    two packed linears and the activation separately)."""

    def __init__(self, hidden: int, columns: int, device=None) -> None:
        super().__init__()
        self.layout = PackedTensorLayout.for_tensor(2 * hidden, columns)
        self.hidden = hidden
        if device is None and torch.cuda.is_available():
            device = torch.device("cuda", torch.cuda.current_device())
        self.register_buffer("packed", torch.zeros(packed_shape(self.layout), dtype=torch.int32, device=device))

    @classmethod
    def from_linears(cls, gate: nn.Linear, up: nn.Linear) -> "PackedSwiGLU":
        if gate.bias is not None or up.bias is not None:
            raise FormatError("a packed linear layer cannot carry a bias")
        if gate.weight.shape != up.weight.shape:
            raise FormatError(f"gate {tuple(gate.weight.shape)} and up {tuple(up.weight.shape)} differ")
        hidden, columns = gate.weight.shape
        return cls(hidden, columns, device=gate.weight.device)

    def load_blocks(self, gate, up, *, validate: bool = True) -> "PackedSwiGLU":
        """Canonical ``(hidden, G, 28)`` blocks of each projection."""
        from .artifact import upload

        def host(blocks):
            return blocks.cpu().numpy() if isinstance(blocks, torch.Tensor) else np.asarray(blocks)

        fused = interleave_gate_up(host(gate), host(up))
        self.packed = upload(fused, self.layout, device=self.packed.device, validate=validate)
        return self

    def load_sidecar(self, path, gate: str, up: str) -> "PackedSwiGLU":
        from .artifact import read_sidecar, sidecar_blocks, sidecar_tensors

        tensors = sidecar_tensors(read_sidecar(path)[1])
        for name in (gate, up):
            if name not in tensors:
                raise FormatError(f"sidecar has no tensor {name!r}")
        return self.load_blocks(sidecar_blocks(path, tensors[gate]), sidecar_blocks(path, tensors[up]))

    def load_safetensors(self, path, gate: str, up: str) -> "PackedSwiGLU":
        from .artifact import safetensors_blocks

        return self.load_blocks(safetensors_blocks(path, gate)[1], safetensors_blocks(path, up)[1])

    def extra_repr(self) -> str:
        return f"{self.layout.columns} -> 2 x {self.hidden} -> {self.hidden}, SiLU(gate) * up"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.layout.columns:
            raise FormatError(f"activations have {x.shape[-1]} columns, expected {self.layout.columns}")
        flat = x.reshape(-1, self.layout.columns)
        return tq1_swiglu_words(self.packed, flat, layout=self.layout).reshape(*x.shape[:-1], self.hidden)


def replace_with_packed(model: nn.Module, *, embedding_dtype: torch.dtype = torch.float16) -> nn.Module:
    """Swap every bias-free ``nn.Linear`` and every ``nn.Embedding`` for its packed twin.

    The packed modules start zero-filled; their weights arrive through
    ``load_blocks``/``load_packed``/``load_weights``.
    """
    for name, child in list(model.named_children()):
        if isinstance(child, nn.Linear) and child.bias is None and child.in_features % 128 == 0:
            setattr(model, name, PackedLinear.from_linear(child))
        elif isinstance(child, nn.Embedding) and child.embedding_dim % 128 == 0:
            setattr(model, name, PackedEmbedding.from_embedding(child, dtype=embedding_dtype))
        else:
            replace_with_packed(child, embedding_dtype=embedding_dtype)
    return model


def load_packed_model(model: nn.Module, path, *, names=None) -> list[str]:
    """Fill every packed module of ``model`` from an artifact: a canonical
    sidecar, or an MLX safetensors file (``.safetensors``). ``names`` maps a
    module path (``layers.0.mlp.down_proj``) to its tensor name in the
    artifact; by default the tensor carries the module path (the MLX
    artifact's convention, src/ternel_mlx/packed_model.py:72-92). Returns the
    module paths loaded; a missing tensor raises FormatError."""
    from pathlib import Path

    safetensors = Path(path).suffix == ".safetensors"
    loaded = []
    for module_path, module in model.named_modules():
        if not isinstance(module, _PackedWeight):
            continue
        tensor = names(module_path) if callable(names) else (names or {}).get(module_path, module_path)
        if safetensors:
            module.load_safetensors(path, tensor)
        else:
            module.load_sidecar(path, tensor)
        loaded.append(module_path)
    return loaded


__all__ = [
    "BLOCK_BYTES",
    "LUT23_MAX_BATCH",
    "PackedEmbedding",
    "PackedLinear",
    "PackedSwiGLU",
    "load_packed_model",
    "matmul_words",
    "packed_matmul",
    "replace_with_packed",
    "select_kernel",
]
