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


# ---------------------------------------------------------------------------
# HF FP8 checkpoints: every quantized Linear is transformers' FP8Linear, the
# layer type the reference compresses (scripts/compress.py:519-528) and runs
# through generate (scripts/inference_llm.py:94-137).

FP8_QUANT_CONFIG = {"quant_method": "fp8", "activation_scheme": "dynamic",
                    "weight_block_size": [128, 128], "modules_to_not_convert": ["lm_head"]}


def _fp8_tiny_config():
    # every projection a multiple of 128 on both sides (128x128 weight scales)
    return transformers.Qwen3Config(
        vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
        num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=128,
        tie_word_embeddings=False)


def _fp8_linear_model(seed=0, dtype=torch.bfloat16):
    """A tiny Qwen3ForCausalLM whose decoder-layer Linears are real
    FP8Linear modules (e4m3fn weight, fp32 weight_scale_inv per 128x128
    block), as transformers builds them from an FP8 checkpoint, and whose
    other parameters are ``dtype``; returns (model, {Linear path: fp8
    bytes})."""
    from transformers.integrations.finegrained_fp8 import FP8Linear

    from ecf8_amd.synth import synthetic_fp8

    torch.manual_seed(seed)
    model = transformers.Qwen3ForCausalLM(_fp8_tiny_config()).to(dtype)
    fp8 = {}
    for li, layer in enumerate(model.model.layers):
        for k, path in enumerate(LINEARS):
            lin = layer.get_submodule(path)
            q = FP8Linear(lin.in_features, lin.out_features, block_size=(128, 128))
            w, s = synthetic_fp8(lin.out_features, lin.in_features, 0.02, seed=seed + li * 10 + k)
            q.weight = torch.nn.Parameter(w, requires_grad=False)
            q.weight_scale_inv = torch.nn.Parameter(s, requires_grad=False)
            layer.set_submodule(path, q)
            fp8[f"model.layers.{li}.{path}"] = w.view(torch.uint8).clone()
    model.config.quantization_config = dict(FP8_QUANT_CONFIG)
    return model, fp8


def _fp8_checkpoint(tmp_path, dtype=torch.bfloat16):
    """(FP8 checkpoint dir, compressed dir, {Linear path: fp8 bytes})."""
    from dfloat.compress import compress_model

    orig_dir, comp_dir = str(tmp_path / "fp8"), str(tmp_path / "fp8-comp")
    model, fp8 = _fp8_linear_model(dtype=dtype)
    model.save_pretrained(orig_dir)
    pattern = compress_model(model, [r"model\.layers\.\d+"], comp_dir,
                             bf16_regex=[r"model\.embed_tokens", r"lm_head"])
    assert pattern["fp8"][r"model\.layers\.\d+"] == list(LINEARS)
    return orig_dir, comp_dir, fp8


def test_compress_model_takes_fp8linear_layers(tmp_path):
    """All seven FP8Linear modules of every decoder layer are compressed
    into the layer's block (their weights removed, the block's buffers
    registered), and the block decodes (oracle) to their FP8 bytes."""
    from transformers.integrations.finegrained_fp8 import FP8Linear

    from dfloat.compress import compress_model, fp8_layers_by_block

    model, fp8 = _fp8_linear_model()
    assert all(type(model.model.layers[0].get_submodule(p)) is FP8Linear for p in LINEARS)
    blocks = fp8_layers_by_block(model, [r"model\.layers\.\d+"])
    assert sorted(blocks) == ["model.layers.0", "model.layers.1"]
    for name, layers in blocks.items():
        assert list(layers) == [f"{name}.{p}" for p in LINEARS]
    compress_model(model, [r"model\.layers\.\d+"], str(tmp_path / "c"))
    for li, layer in enumerate(model.model.layers):
        for path in LINEARS:
            # the compressed model drops the Linear modules themselves, as the
            # reference does (scripts/compress.py:587-602); the loader takes
            # them, scales included, from the original FP8 checkpoint
            parent, attr = path.split(".")
            assert not hasattr(layer.get_submodule(parent), attr)
        flat = oc.decode(layer.luts.numpy(), layer.encoded.numpy(),
                         layer.packed_other_4bits.numpy(), layer.output_positions.numpy(),
                         layer.gaps.numpy())
        for path, part in zip(LINEARS, np.split(flat, layer.split_positions)):
            assert np.array_equal(part, fp8[f"model.layers.{li}.{path}"].numpy().reshape(-1)), path


def test_fp8_checkpoint_compresses_and_keeps_its_quantization_config(tmp_path):
    """The compressed HF directory keeps the FP8 checkpoint's
    quantization_config beside dfloat_config and holds nothing of a
    compressed Linear: weights and scales are the original checkpoint's."""
    from safetensors.torch import load_file

    _orig, comp_dir, _fp8 = _fp8_checkpoint(tmp_path)
    with open(os.path.join(comp_dir, "config.json")) as f:
        cfg = json.load(f)
    assert cfg["quantization_config"]["quant_method"] == "fp8"
    assert cfg["dfloat_config"]["threads_per_block"] == 512
    names = set()
    for fn in os.listdir(comp_dir):
        if fn.endswith(".safetensors"):
            names |= set(load_file(os.path.join(comp_dir, fn)))
    for li in range(2):
        for path in LINEARS:
            assert f"model.layers.{li}.{path}.weight" not in names
            assert f"model.layers.{li}.{path}.weight_scale_inv" not in names
        assert f"model.layers.{li}.encoded" in names


def test_a_matching_block_without_fp8_layers_is_refused(tmp_path):
    """A block the patterns select that holds no e4m3fn layer raises instead
    of being written as an uncompressed 'compressed' checkpoint."""
    from dfloat.compress import compress_model, fp8_layers_by_block

    model = transformers.Qwen3ForCausalLM(_tiny_config()).to(torch.bfloat16)
    with pytest.raises(ValueError, match="hold no float8_e4m3fn"):
        fp8_layers_by_block(model, [r"model\.layers\.\d+"])
    with pytest.raises(ValueError, match="no module of the model matches"):
        compress_model(model, [r"model\.decoder\.\d+"], str(tmp_path / "x"))


def test_fp8linear_binding_refuses_the_cpu():
    """The engine's FP8Linear forward has no CPU path."""
    from ecf8_amd._lib import ECF8Error
    from ecf8_amd.hf_fp8 import bind_fp8_linears

    model, _ = _fp8_linear_model()
    assert bind_fp8_linears(model) == 14
    assert bind_fp8_linears(model) == 14  # idempotent
    with pytest.raises(ECF8Error, match="no CPU path"):
        model.model.layers[0].self_attn.q_proj(torch.zeros(1, 256, dtype=torch.bfloat16))


@pytest.mark.gpu
def test_dfloat_model_generates_like_the_fp8_model(tmp_path, cuda_device):
    """The reference's inference flow on an HF FP8 checkpoint: transformers
    loads it with FP8Linear modules, ``DFloatModel.from_pretrained`` swaps
    their weights for the compressed blocks and their forward for the
    engine's FP8 linear, and ``generate`` gives the tokens and logits of the
    same checkpoint loaded uncompressed with the same binding (the decoded
    weights are bit-exact and every kernel is deterministic, so equality is
    exact).  The model's other parts run in float32: torch's batched bf16
    products with a transposed operand are avoided on this GPU."""
    from transformers.integrations.finegrained_fp8 import FP8Linear

    from dfloat.run.run import DFloatModel, TensorManager
    from ecf8_amd.hf_fp8 import bind_fp8_linears

    orig_dir, comp_dir, fp8 = _fp8_checkpoint(tmp_path, dtype=torch.float32)
    TensorManager.clear_device()
    ref = transformers.AutoModelForCausalLM.from_pretrained(
        orig_dir, dtype=torch.float32, attn_implementation="eager").to(cuda_device).eval()
    assert type(ref.model.layers[0].self_attn.q_proj) is FP8Linear
    assert bind_fp8_linears(ref) == 14
    comp = DFloatModel.from_pretrained(comp_dir, "local/tiny-fp8-DF6.5", orig_dir,
                                       device=str(cuda_device), torch_dtype=torch.float32,
                                       attn_implementation="eager")
    comp.eval()
    layer0 = comp.model.layers[0]
    assert type(layer0.self_attn.q_proj) is FP8Linear and len(layer0._forward_pre_hooks) == 1

    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 512, (3, 24), generator=g).to(cuda_device)
    mask = torch.ones_like(ids)
    with torch.no_grad():
        logits_ref = ref(input_ids=ids, attention_mask=mask).logits
        logits_comp = comp(input_ids=ids, attention_mask=mask).logits
        torch.cuda.synchronize()
        assert torch.isfinite(logits_ref).all()
        assert torch.equal(logits_ref, logits_comp)
        # the injected weights are the checkpoint's FP8 bytes
        for li, layer in enumerate(comp.model.layers):
            for path in LINEARS:
                w = layer.get_submodule(path).weight
                if li == len(comp.model.layers) - 1:  # the shared buffer holds the last layer
                    assert torch.equal(w.view(torch.uint8).cpu(), fp8[f"model.layers.{li}.{path}"])
        kw = dict(attention_mask=mask, max_new_tokens=8, do_sample=False, pad_token_id=0)
        out_ref = ref.generate(ids, **kw)
        out_comp = comp.generate(ids, **kw)
    torch.cuda.synchronize()
    assert out_ref.shape[0] == 3 and out_ref.shape[1] > 24
    assert torch.equal(out_ref, out_comp)
