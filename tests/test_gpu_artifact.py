"""Artifact loaders end to end on the GPU: tensors read from a canonical sidecar
or an MLX safetensors file land as the same packed words as the blocks they
hold, pass the on-GPU scan, and compute the same products."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import tq1_oracle as O
from tests.gpu_util import layout, pack, random_blocks, to_dev
from ternel_amd.artifact import load_safetensors_tensor, load_sidecar_tensor, read_sidecar, save_safetensors, \
    sidecar_tensors, write_sidecar
from ternel_amd.format import FormatError
from ternel_amd.kernels import tq1_matmul_words
from ternel_amd.modules import PackedEmbedding, PackedLinear, load_packed_model, replace_with_packed

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(("rows", "columns"), ((300, 640), (1024, 5120), (256, 17408)))
def test_sidecar_tensor_loads_to_the_same_packed_words(tmp_path, rows: int, columns: int) -> None:
    blocks = random_blocks(rows, columns, seed=rows + columns)
    path = tmp_path / "model.tq1"
    write_sidecar(path, {"filler": random_blocks(3, 128, seed=1), "w": blocks})
    lay, packed = load_sidecar_tensor(path, "w")
    assert (lay.rows, lay.columns) == (rows, columns)
    assert torch.equal(packed, pack(blocks))
    x = np.random.default_rng(rows).normal(0, 1, size=(1, columns)).astype(np.float32)
    got = tq1_matmul_words(packed, to_dev(x), layout=lay).cpu().numpy()
    np.testing.assert_array_equal(got, tq1_matmul_words(pack(blocks), to_dev(x), layout=layout(rows, columns)).cpu().numpy())
    oracle = O.oracle_matmul(blocks, x, rows=rows, columns=columns)
    assert O.compare(got, oracle)["normalised_max_abs_error"] < 1e-3


@pytest.mark.parametrize(("position", "value", "message"), ((2, 243, "regular=1"), (27, 27, "tail=1")))
def test_sidecar_with_an_illegal_code_byte_fails_the_load(tmp_path, position: int, value: int, message: str) -> None:
    blocks = random_blocks(64, 256, seed=3)
    path = tmp_path / "model.tq1"
    write_sidecar(path, {"w": blocks})
    entry = sidecar_tensors(read_sidecar(path)[1])["w"]
    raw = bytearray(path.read_bytes())
    raw[entry.offset + 28 * 77 + position] = value  # block 77
    path.write_bytes(bytes(raw))
    with pytest.raises(FormatError, match=f"out-of-range base-3 bytes: .*{message}"):
        load_sidecar_tensor(path, "w")
    with pytest.raises(FormatError, match=message):
        PackedLinear.from_sidecar(path, "w")


def test_packed_layers_from_either_artifact_match_loaded_blocks(tmp_path) -> None:
    blocks = random_blocks(512, 1024, seed=5)
    sidecar, st = tmp_path / "model.tq1", tmp_path / "model.safetensors"
    write_sidecar(sidecar, {"blk.0.ffn_up.weight": blocks})
    save_safetensors(st, {"model.layers.0.mlp.up_proj": blocks})
    direct = PackedLinear(layout(512, 1024))
    direct.load_blocks(blocks)
    x = torch.from_numpy(np.random.default_rng(5).normal(0, 1, size=(3, 1024)).astype(np.float16)).cuda()
    want = direct(x)
    for layer in (PackedLinear.from_sidecar(sidecar, "blk.0.ffn_up.weight"),
                  PackedLinear.from_safetensors(st, "model.layers.0.mlp.up_proj")):
        assert torch.equal(layer.packed, direct.packed)
        assert torch.equal(layer(x), want)
    lay, packed = load_safetensors_tensor(st, "model.layers.0.mlp.up_proj")
    assert lay.tile == 256 and torch.equal(packed, direct.packed)


def test_embedding_rows_from_a_sidecar_are_exact(tmp_path) -> None:
    blocks = random_blocks(300, 256, seed=7)
    path = tmp_path / "model.tq1"
    write_sidecar(path, {"token_embd.weight": blocks})
    table = PackedEmbedding.from_sidecar(path, "token_embd.weight", dtype=torch.float16)
    ids = torch.tensor([[0, 299], [17, 300]], device="cuda")
    rows = table(ids).float().cpu().numpy()
    dense = O.dense_weights(blocks, rows=300, columns=256).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(rows[0, 0], dense[0])
    np.testing.assert_array_equal(rows[0, 1], dense[299])
    np.testing.assert_array_equal(rows[1, 0], dense[17])
    np.testing.assert_array_equal(rows[1, 1], np.zeros(256, dtype=np.float32))  # outside the table


def test_a_swapped_model_loads_every_packed_module(tmp_path) -> None:
    model = nn.Sequential(nn.Embedding(300, 256), nn.Linear(256, 512, bias=False), nn.Linear(512, 256, bias=False))
    replace_with_packed(model)
    weights = {"0": random_blocks(300, 256, seed=11), "1": random_blocks(512, 256, seed=12),
               "2": random_blocks(256, 512, seed=13)}
    for path, names in ((tmp_path / "m.safetensors", None),
                        (tmp_path / "m.tq1", {"0": "token_embd.weight", "1": "blk.0.ffn_up.weight",
                                              "2": "blk.0.ffn_down.weight"})):
        if path.suffix == ".safetensors":
            save_safetensors(path, weights)
        else:
            write_sidecar(path, {names[k]: v for k, v in weights.items()})
        assert load_packed_model(model, path, names=names) == ["0", "1", "2"]
        for key, module in model.named_children():
            assert torch.equal(module.packed, pack(weights[key])), key
    with pytest.raises(FormatError, match="no tensor"):
        load_packed_model(model, tmp_path / "m.tq1")  # sidecar names differ from module paths
