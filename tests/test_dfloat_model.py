"""DFloatModel.from_pretrained (dfloat/run/run.py:483-566) over a real
transformers model, on the CPU: a tiny random Qwen3ForCausalLM is saved
locally, its decoder layers' Linears are given FP8 weights and compressed
by ``compress_model``, which writes the reference's layout through
``save_pretrained`` (config.json carrying ``dfloat_config``,
pattern_dict.json, the compressed safetensors); the loader registers
every layer's compressed block on a fresh instance of the original model.
Each registered block decodes (oracle) to the FP8 weights that were
compressed, and the dense weights it replaces are gone."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import codec as oc

transformers = pytest.importorskip("transformers")

LINEARS = ("mlp.down_proj", "mlp.gate_proj", "mlp.up_proj", "self_attn.k_proj",
           "self_attn.o_proj", "self_attn.q_proj", "self_attn.v_proj")


def _tiny_config():
    return transformers.Qwen3Config(
        vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
        num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=64,
        tie_word_embeddings=False)


def _checkpoint(tmp_path):
    """(original model dir, compressed dir, the original model, its FP8
    weights by Linear path)."""
    from dfloat.compress import compress_model
    from ecf8_amd.synth import synthetic_fp8

    torch.manual_seed(0)
    orig_dir, comp_dir = str(tmp_path / "orig"), str(tmp_path / "comp")
    model = transformers.Qwen3ForCausalLM(_tiny_config()).to(torch.bfloat16)
    model.save_pretrained(orig_dir)

    # the FP8 weights of every decoder-layer Linear, then compress as the
    # reference does for `model.layers.N`
    fp8 = {}
    for li, layer in enumerate(model.model.layers):
        for k, path in enumerate(LINEARS):
            lin = layer.get_submodule(path)
            w, _ = synthetic_fp8(lin.out_features, lin.in_features, 0.02, seed=li * 10 + k)
            lin.weight = torch.nn.Parameter(w, requires_grad=False)
            fp8[f"model.layers.{li}.{path}"] = w.view(torch.uint8).clone()
    pattern = compress_model(model, [r"model\.layers\.\d+"], comp_dir, n_workers=2,
                             bf16_regex=[r"model\.embed_tokens", r"lm_head"])
    assert pattern["fp8"][r"model\.layers\.\d+"] == list(LINEARS)
    # the compressor writes the reference's layout for a transformers model
    # (scripts/compress.py:668-677): config.json carries dfloat_config, and
    # no separate dfloat_config.json is written
    with open(os.path.join(comp_dir, "config.json")) as f:
        cfg = json.load(f)
    assert cfg["dfloat_config"] == {"version": "0.2.0", "threads_per_block": 512,
                                    "bytes_per_thread": 8}
    assert not os.path.exists(os.path.join(comp_dir, "dfloat_config.json"))
    with open(os.path.join(comp_dir, "pattern_dict.json")) as f:
        assert json.load(f) == {"fp8": {r"model\.layers\.\d+": list(LINEARS)},
                                "bf16": {r"model\.embed_tokens": [], r"lm_head": []}}
    return orig_dir, comp_dir, model, fp8


def test_dfloat_model_loads_a_compressed_transformers_checkpoint(tmp_path):
    from dfloat.run.run import DFloatModel

    orig_dir, comp_dir, model, fp8 = _checkpoint(tmp_path)
    loaded = DFloatModel.from_pretrained(comp_dir, "local/tiny-DF6.5", orig_dir, device="cpu")
    for li, layer in enumerate(loaded.model.layers):
        assert len(layer._forward_pre_hooks) == 1
        assert [type(m).__name__ for m in layer.weight_injection_modules] == ["Linear"] * 7
        for path in LINEARS:
            assert "weight" not in layer.get_submodule(path)._parameters
        flat = oc.decode(layer.luts.numpy(), layer.encoded.numpy(),
                         layer.packed_other_4bits.numpy(), layer.output_positions.numpy(),
                         layer.gaps.numpy())
        for path, part in zip(LINEARS, np.split(flat, layer.split_positions)):
            assert np.array_equal(part, fp8[f"model.layers.{li}.{path}"].numpy().reshape(-1)), path
    # the parameters outside the blocks come from the compressed checkpoint
    assert torch.equal(loaded.lm_head.weight, model.lm_head.weight)
    assert torch.equal(loaded.model.embed_tokens.weight, model.model.embed_tokens.weight)


@pytest.mark.gpu
def test_dfloat_model_hooks_inject_bit_exact_weights(tmp_path, cuda_device):
    """The same checkpoint loaded onto the GPU: each decoder layer's
    forward-pre-hook decodes its block with the HIP kernel and injects
    views equal to the FP8 weights that were compressed."""
    from dfloat.run.run import DFloatModel, TensorManager

    orig_dir, comp_dir, _model, fp8 = _checkpoint(tmp_path)
    TensorManager.clear_device()
    loaded = DFloatModel.from_pretrained(comp_dir, "local/tiny-DF6.5", orig_dir,
                                         device=str(cuda_device))
    for li, layer in enumerate(loaded.model.layers):
        for hook in layer._forward_pre_hooks.values():
            hook(layer, None)
        torch.cuda.synchronize()
        for path in LINEARS:
            w = layer.get_submodule(path).weight
            assert w.is_cuda and w.dtype == torch.float8_e4m3fn
            assert torch.equal(w.view(torch.uint8).cpu(), fp8[f"model.layers.{li}.{path}"]), path
