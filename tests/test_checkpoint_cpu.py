"""Checkpoint ingestion (CPU): MXFP4 linears read tensor by tensor from safetensors files, merged
parts concatenated along N, both tensor namings, shape checks before anything reaches a GPU."""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from vllm_sly_radiance_amd import checkpoint as CK
from vllm_sly_radiance_amd import synthetic


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def write_sharded(tmp_path, tensors_per_shard):
    """Shards model-0000i-of-0000n.safetensors plus model.safetensors.index.json."""
    wm = {}
    n = len(tensors_per_shard)
    for i, tens in enumerate(tensors_per_shard):
        fn = f"model-{i + 1:05d}-of-{n:05d}.safetensors"
        save_file(tens, os.path.join(tmp_path, fn))
        wm.update({k: fn for k in tens})
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)


@pytest.fixture
def ckpt(tmp_path):
    K = 512
    g, gs = synthetic.weights(48, K, 1)
    u, us = synthetic.weights(32, K, 2)
    d, ds = synthetic.weights(16, 1024, 3)
    write_sharded(tmp_path, [
        {"model.layers.0.mlp.gate_proj.weight_packed": t(g),       # compressed-tensors naming
         "model.layers.0.mlp.gate_proj.weight_scale": t(gs)},
        {"model.layers.0.mlp.up_proj.weight_packed": t(u),
         "model.layers.0.mlp.up_proj.weight_scale": t(us),
         "model.layers.0.mlp.down_proj.weight": t(d),               # Quark naming
         "model.layers.0.mlp.down_proj.weight_scale": t(ds)},
    ])
    return tmp_path, (g, gs, u, us, d, ds)


def test_merged_parts_concatenate_along_n(ckpt):
    path, (g, gs, u, us, _, _) = ckpt
    idx = CK.CheckpointIndex(str(path))
    w, s = CK.read_mxfp4_linear(idx, "model.layers.0.mlp", ["gate_proj", "up_proj"])
    assert w.dtype == torch.uint8 and tuple(w.shape) == (80, 256)
    assert np.array_equal(w.numpy(), np.concatenate([g, u], 0))
    assert np.array_equal(s.numpy(), np.concatenate([gs, us], 0))


def test_quark_naming_and_single_linear(ckpt):
    path, (*_, d, ds) = ckpt
    idx = CK.CheckpointIndex(str(path))
    w, s = CK.read_mxfp4_linear(idx, "model.layers.0.mlp.down_proj")
    assert np.array_equal(w.numpy(), d) and np.array_equal(s.numpy(), ds)


def test_single_file_and_unindexed_directory(tmp_path):
    w, ws = synthetic.weights(16, 256, 4)
    save_file({"lin.weight": t(w), "lin.weight_scale": t(ws)},
              os.path.join(tmp_path, "a.safetensors"))
    for p in (str(tmp_path), os.path.join(tmp_path, "a.safetensors")):
        got, gs = CK.read_mxfp4_linear(CK.CheckpointIndex(p), "lin")
        assert np.array_equal(got.numpy(), w) and np.array_equal(gs.numpy(), ws)


def test_load_linear_sets_the_plugin_parameters(ckpt):
    path, (g, gs, u, us, _, _) = ckpt
    layer = torch.nn.Module()
    CK.load_linear(layer, CK.CheckpointIndex(str(path)), "model.layers.0.mlp",
                   ["gate_proj", "up_proj"], device="cpu")
    assert isinstance(layer.weight, torch.nn.Parameter) and not layer.weight.requires_grad
    assert tuple(layer.weight.shape) == (80, 256) and tuple(layer.weight_scale.shape) == (80, 16)


def test_shape_and_name_errors(tmp_path):
    a, as_ = synthetic.weights(16, 512, 5)
    b, bs = synthetic.weights(16, 256, 6)               # a different K
    save_file({"m.a.weight": t(a), "m.a.weight_scale": t(as_),
               "m.b.weight": t(b), "m.b.weight_scale": t(bs),
               "m.c.weight": t(a.copy()), "m.c.weight_scale": t(as_[:, :8].copy()),
               "m.f.weight": t(a.astype(np.float32)), "m.f.weight_scale": t(as_.copy())},
              os.path.join(tmp_path, "x.safetensors"))
    idx = CK.CheckpointIndex(str(tmp_path))
    with pytest.raises(RuntimeError, match="differs"):
        CK.read_mxfp4_linear(idx, "m", ["a", "b"])
    with pytest.raises(RuntimeError, match="does not match"):
        CK.read_mxfp4_linear(idx, "m.c")
    with pytest.raises(RuntimeError, match="uint8"):
        CK.read_mxfp4_linear(idx, "m.f")
    with pytest.raises(KeyError):
        CK.read_mxfp4_linear(idx, "m.missing")
    with pytest.raises(RuntimeError, match="no safetensors"):
        CK.CheckpointIndex(str(tmp_path / "empty_dir_that_does_not_exist"))
