"""MLX quantized safetensors checkpoints -> verify modules (dflash-mlx_amd/loader.py).

Synthetic checkpoints in the MLX format are written here with the oracle's
packer; the loader must hand the stored words over unchanged (the kernels'
layout is the file's layout), apply the config's per-module quantization,
find sharded files through the index the way the reference does
(dflash_mlx/runtime/loading.py:124-158) and reject inconsistent checkpoints.
The GPU test runs the loaded modules against the oracle.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

import oracle

from .conftest import from_dev, to_dev  # noqa: F401  (GPU test)


def _quantized(rng, N, K, gs, bits):
    codes = rng.integers(0, 2 ** bits, size=(N, K))
    w = oracle.pack(codes, bits)
    s = oracle.f32_to_bf16_bits((rng.random((N, K // gs)) * 0.02 + 0.001).astype(np.float32))
    b = oracle.f32_to_bf16_bits((rng.standard_normal((N, K // gs)) * 0.05).astype(np.float32))
    return codes, w, s, b


def _torch_tensors(w, s, b):
    import torch

    return (torch.from_numpy(w.astype(np.uint32)),
            torch.from_numpy(s.view(np.int16)).view(torch.bfloat16),
            torch.from_numpy(b.view(np.int16)).view(torch.bfloat16))


def _write_checkpoint(tmp_path, sharded=True):
    """Two layers: q_proj / k_proj 4-bit gs64, down_proj 8-bit gs32 by a
    per-module override, gate_proj left unquantized (``false``)."""
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(11)
    spec = {}
    shards = [{}, {}]
    for layer in range(2):
        for proj, (N, K, gs, bits) in {"self_attn.q_proj": (128, 256, 64, 4),
                                       "self_attn.k_proj": (64, 256, 64, 4),
                                       "mlp.down_proj": (96, 512, 32, 8)}.items():
            path = f"model.layers.{layer}.{proj}"
            codes, w, s, b = _quantized(rng, N, K, gs, bits)
            wt, st, bt = _torch_tensors(w, s, b)
            shard = shards[layer] if sharded else shards[0]
            shard[f"{path}.weight"], shard[f"{path}.scales"], shard[f"{path}.biases"] = wt, st, bt
            spec[path] = (codes, w, s, b, gs, bits)
        shards[layer if sharded else 0][f"model.layers.{layer}.mlp.gate_proj.weight"] = \
            torch.zeros((32, 256), dtype=torch.bfloat16)
    q = {"group_size": 64, "bits": 4}
    for layer in range(2):
        q[f"model.layers.{layer}.mlp.down_proj"] = {"group_size": 32, "bits": 8}
        q[f"model.layers.{layer}.mlp.gate_proj"] = False
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "qwen3", "quantization": q}))
    if sharded:
        names = {}
        for i, shard in enumerate(shards):
            fname = f"model-0000{i + 1}-of-00002.safetensors"
            save_file(shard, str(tmp_path / fname))
            names.update({k: fname for k in shard})
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": names}))
    else:
        save_file(shards[0], str(tmp_path / "model.safetensors"))
    return spec


@pytest.mark.parametrize("sharded", [True, False])
def test_loads_words_unchanged_with_per_module_quantization(tmp_path, sharded):
    import torch

    from dflash_mlx_amd import loader
    from dflash_mlx_amd.verify_linear import VerifyQuantizedLinear

    spec = _write_checkpoint(tmp_path, sharded=sharded)
    mods = loader.load_quantized_linears(tmp_path, device="cpu")
    assert sorted(mods) == sorted(spec)
    for path, (codes, w, s, b, gs, bits) in spec.items():
        m = mods[path]
        assert isinstance(m, VerifyQuantizedLinear)
        assert (m.group_size, m.bits, m.mode) == (gs, bits, "affine")
        got_w = m.weight.numpy().astype(np.uint32)
        assert np.array_equal(got_w, w.astype(np.uint32))             # no repacking
        assert np.array_equal(oracle.unpack(got_w, bits), codes)  # k order pinned
        assert np.array_equal(m.scales.view(torch.int16).numpy().view(np.uint16), s)
        assert np.array_equal(m.biases.view(torch.int16).numpy().view(np.uint16), b)
    assert not any("gate_proj" in p for p in mods)


def test_shard_discovery_follows_the_index(tmp_path):
    from dflash_mlx_amd import loader

    _write_checkpoint(tmp_path, sharded=True)
    files = loader.weight_files(tmp_path)
    assert [f.name for f in files] == ["model-00001-of-00002.safetensors",
                                       "model-00002-of-00002.safetensors"]
    (tmp_path / "model.safetensors.index.json").write_text("{not json")
    with pytest.raises(ValueError, match="Invalid safetensors index JSON"):
        loader.weight_files(tmp_path)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": []}))
    with pytest.raises(ValueError, match="weight_map"):
        loader.weight_files(tmp_path)


def test_quantization_config_rules():
    from dflash_mlx_amd.loader import quantization_for

    cfg = {"quantization": {"group_size": 32, "bits": 4, "a.b": {"bits": 8},
                            "a.c": False, "a.d": {"group_size": 128, "mode": "mxfp4"}}}
    assert quantization_for(cfg, "x.y") == (32, 4, "affine")
    assert quantization_for(cfg, "a.b") == (32, 8, "affine")
    assert quantization_for(cfg, "a.c") is None
    assert quantization_for(cfg, "a.d") == (128, 4, "mxfp4")
    assert quantization_for({"quantization_config": {"bits": 8}}, "z") == (64, 8, "affine")
    assert quantization_for({}, "z") is None


def test_rejects_inconsistent_checkpoints(tmp_path):
    import torch
    from safetensors.torch import save_file

    from dflash_mlx_amd import loader

    rng = np.random.default_rng(3)
    _, w, s, b = _quantized(rng, 64, 256, 64, 4)
    wt, st, bt = _torch_tensors(w, s, b)
    save_file({"l.weight": wt, "l.scales": st, "l.biases": bt}, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="no quantization entry"):
        loader.load_quantized_linears(tmp_path, device="cpu")
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"group_size": 32, "bits": 4}}))
    with pytest.raises(ValueError, match="do not match"):
        loader.load_quantized_linears(tmp_path, device="cpu")
    save_file({"l.weight": wt, "l.scales": st}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"group_size": 64, "bits": 4}}))
    with pytest.raises(ValueError, match="biases"):
        loader.load_quantized_linears(tmp_path, device="cpu")
    save_file({"l.weight": wt.to(torch.int64), "l.scales": st, "l.biases": bt},
              str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="uint32"):
        loader.load_quantized_linears(tmp_path, device="cpu")


def test_install_into_module_tree(tmp_path):
    from torch import nn

    from dflash_mlx_amd import loader

    _write_checkpoint(tmp_path, sharded=True)
    mods = loader.load_quantized_linears(tmp_path, device="cpu",
                                         include=["model.layers.1."])
    assert sorted(mods) == ["model.layers.1.mlp.down_proj", "model.layers.1.self_attn.k_proj",
                            "model.layers.1.self_attn.q_proj"]

    class Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj, self.k_proj = nn.Linear(256, 128), nn.Linear(256, 64)

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = Attn()

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList([Layer(), Layer()])

    root = nn.Module()
    root.model = Model()
    assert loader.install_quantized_linears(root, mods) == 2   # no mlp in this tree
    assert root.model.layers[1].self_attn.q_proj is mods["model.layers.1.self_attn.q_proj"]
    assert isinstance(root.model.layers[0].self_attn.q_proj, nn.Linear)


@pytest.mark.gpu
def test_loaded_modules_run_the_verify_kernels(tmp_path, dev):
    import torch

    from dflash_mlx_amd import loader

    spec = _write_checkpoint(tmp_path, sharded=True)
    mods = loader.load_quantized_linears(tmp_path, device=dev)
    rng = np.random.default_rng(5)
    for path, (codes, w, s, b, gs, bits) in spec.items():
        K = codes.shape[1]
        x = oracle.f32_to_bf16_bits(rng.standard_normal((16, K)).astype(np.float32))
        y = mods[path](to_dev(x, "bf16", dev).reshape(1, 16, K))
        torch.cuda.synchronize()
        want = oracle.quantized_matmul(x, w, s, b, group_size=gs, bits=bits, dtype="bf16")
        got = oracle.to_f32(from_dev(y.reshape(16, -1), "bf16"), "bf16").astype(np.float64)
        _, rel = oracle.parity_metrics(got, want)
        assert rel <= 1e-2, f"{path}: {rel}"
