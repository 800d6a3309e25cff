"""Compressed checkpoints in the reference's on-disk layout
(scripts/compress.py:490-680, dfloat/run/run.py:158-458): compress a small
model block by block, save, load into a fresh instance, and check the
stored tensors (CPU, against the oracle's decode) and the weights the
decode hook injects (GPU, bit-exact)."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import codec as oc

LINEARS = {  # (out, in) per linear of a block, Qwen3-shaped names
    "mlp.down_proj": (128, 384),
    "mlp.gate_proj": (384, 128),
    "mlp.up_proj": (384, 128),
    "self_attn.k_proj": (128, 128),
    "self_attn.o_proj": (256, 128),
    "self_attn.q_proj": (256, 128),
    "self_attn.v_proj": (128, 128),
}


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = nn.Module()
        self.mlp = nn.Module()
        self.input_layernorm = nn.LayerNorm(128)
        for path, (o, i) in LINEARS.items():
            parent, name = path.split(".")
            setattr(getattr(self, parent), name, nn.Linear(i, o, bias=False))

    def forward(self, x):
        return self.input_layernorm(x)


class _Model(nn.Module):
    def __init__(self, n_layers=3):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList(_Layer() for _ in range(n_layers))
        self.lm_head = nn.Linear(128, 64, bias=False)

    def forward(self, x):
        for layer in self.model.layers:
            x = layer(x)
        return x


def _fp8_model(seed=0):
    from ecf8_amd.synth import synthetic_fp8

    m = _Model()
    originals = {}
    for li, layer in enumerate(m.model.layers):
        for k, path in enumerate(sorted(LINEARS)):
            o, i = LINEARS[path]
            w, _ = synthetic_fp8(o, i, 0.02, seed=seed * 100 + li * 10 + k)
            lin = layer.get_submodule(path)
            lin.weight = nn.Parameter(w, requires_grad=False)
            originals[f"model.layers.{li}.{path}"] = w.view(torch.uint8).clone()
    return m, originals


@pytest.fixture(scope="module")
def saved(tmp_path_factory):
    from dfloat.compress import compress_model

    d = str(tmp_path_factory.mktemp("ckpt"))
    m, originals = _fp8_model()
    pattern = compress_model(m, [r"model\.layers\.\d+"], d, bf16_regex=[r"lm_head"])
    return d, pattern, originals


def test_parallel_compression_writes_the_same_checkpoint(saved, tmp_path):
    """Blocks compressed in a thread pool (the reference's parallel path)
    give byte-identical block files and the same pattern dict."""
    from safetensors.torch import load_file

    from dfloat.compress import compress_model

    d0, pattern0, _ = saved
    m, _ = _fp8_model()
    d1 = str(tmp_path)
    pattern1 = compress_model(m, [r"model\.layers\.\d+"], d1, bf16_regex=[r"lm_head"],
                              n_workers=3)
    assert pattern1 == pattern0
    names = sorted(f for f in os.listdir(os.path.join(d0, "cache")) if f.endswith(".safetensors"))
    assert names == sorted(f for f in os.listdir(os.path.join(d1, "cache"))
                           if f.endswith(".safetensors"))
    for f in names:
        a, b = load_file(os.path.join(d0, "cache", f)), load_file(os.path.join(d1, "cache", f))
        assert sorted(a) == sorted(b)
        for k in a:
            assert torch.equal(a[k], b[k]), (f, k)
    s0, s1 = (load_file(os.path.join(d, "model.safetensors")) for d in (d0, d1))
    assert sorted(s0) == sorted(s1)
    compressed = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps",
                  "split_positions")
    keys = [k for k in s0 if k.rsplit(".", 1)[-1] in compressed]  # the rest is random init
    assert len(keys) == 3 * len(compressed)
    for k in keys:
        assert torch.equal(s0[k], s1[k]), k


def test_checkpoint_files_follow_the_reference_layout(saved):
    from safetensors.torch import load_file

    d, pattern, _ = saved
    # a module with neither a Hugging Face config nor a pipeline pattern gets
    # the whole state dict in one file
    assert sorted(f for f in os.listdir(d) if not os.path.isdir(os.path.join(d, f))) == [
        "dfloat_config.json", "entropy.csv", "model.safetensors", "pattern_dict.json"]
    with open(os.path.join(d, "entropy.csv")) as f:
        rows = f.read().split()
    assert rows[0] == "block_name,entropy"
    assert [r.split(",")[0] for r in rows[1:]] == [f"model.layers.{i}" for i in range(3)]
    assert all(1.0 < float(r.split(",")[1]) < 4.0 for r in rows[1:])
    assert json.load(open(os.path.join(d, "pattern_dict.json"))) == {
        "fp8": {r"model\.layers\.\d+": sorted(LINEARS)}, "bf16": {"lm_head": []}}
    cfg = json.load(open(os.path.join(d, "dfloat_config.json")))
    assert cfg["threads_per_block"] == 512 and cfg["bytes_per_thread"] == 8
    t = load_file(os.path.join(d, "model.safetensors"))
    for li in range(3):
        p = f"model.layers.{li}."
        assert t[p + "luts"].dtype == torch.uint8 and t[p + "luts"].shape[1] == 256
        assert t[p + "output_positions"].dtype == torch.uint8  # u8 view of u64
        assert t[p + "split_positions"].dtype == torch.int64
        assert not any(k.startswith(p + "mlp.") or k.startswith(p + "self_attn.") for k in t)
        assert p + "input_layernorm.weight" in t


def test_stored_blocks_decode_to_the_original_weights_on_cpu(saved):
    from safetensors.torch import load_file

    d, _, originals = saved
    t = load_file(os.path.join(d, "model.safetensors"))
    for li in range(3):
        p = f"model.layers.{li}."
        flat = oc.decode(t[p + "luts"].numpy(), t[p + "encoded"].numpy(),
                         t[p + "packed_other_4bits"].numpy(), t[p + "output_positions"].numpy(),
                         t[p + "gaps"].numpy())
        parts = np.split(flat, t[p + "split_positions"].numpy())
        for path, part in zip(sorted(LINEARS), parts):
            assert np.array_equal(part, originals[p + path].numpy().reshape(-1))


def test_load_registers_buffers_hooks_and_removes_weights(saved):
    from dfloat.run.run import load_compressed_model

    d, _, _ = saved
    fresh = _Model()
    load_compressed_model(fresh, d)
    for layer in fresh.model.layers:
        assert layer.luts.dtype == torch.uint8
        assert len(layer._forward_pre_hooks) == 1
        assert [type(m) for m in layer.weight_injection_modules] == [nn.Linear] * 7
        for path in LINEARS:
            assert "weight" not in layer.get_submodule(path)._parameters
    assert "weight" in fresh.lm_head._parameters


@pytest.mark.gpu
def test_loaded_checkpoint_injects_bit_exact_weights(saved, cuda_device):
    from dfloat.run.run import TensorManager, load_compressed_model

    d, _, originals = saved
    fresh = load_compressed_model(_Model(), d, parallel=True).to(cuda_device)
    TensorManager.clear_device()
    for li, layer in enumerate(fresh.model.layers):
        layer(torch.zeros(2, 128, device=cuda_device))
        torch.cuda.synchronize()
        for path in LINEARS:
            w = layer.get_submodule(path).weight
            assert w.dtype == torch.float8_e4m3fn and tuple(w.shape) == LINEARS[path]
            got = w.view(torch.uint8).cpu()
            assert torch.equal(got, originals[f"model.layers.{li}.{path}"])
