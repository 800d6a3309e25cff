"""The reference's Python API as its callers use it (CPU).

* the import statements of the reference's own scripts run unchanged
  (scripts/inference_llm.py:9-12, scripts/compress.py:51-62,
  scripts/inference_dfsyn.py:11) and resolve to this package;
* the block patterns of dfloat.const cut the modules the reference cuts,
  checked on module names of the model families (not by restating the
  regexes);
* a DiffSynth-layout checkpoint (one safetensors per block,
  scripts/compress.py:614-624) written by compress_model loads through
  DFloatDiffSynthModelFP8.from_pretrained into a fresh pipeline, and every
  registered block decodes (oracle) to the FP8 weights compressed.
"""

from __future__ import annotations

import json
import os
import re

import numpy as np
import pytest
import torch

from oracle import codec as oc

# verbatim import lines of the reference's scripts
_IMPORTS = {
    "scripts/inference_llm.py:9-12":
        "from dfloat.run import DFloatModel, get_dfloat_model_name_or_path\n",
    "scripts/compress.py:51-62": (
        "from dfloat.const import get_fp8_pattern_dict\n"
        "from dfloat.run import _decode, get_dfloat_model_name_or_path\n"
        "from dfloat.utils import (\n"
        "    encode_exponents_for_cuda,\n"
        "    find_layers_by_data_type_and_layer_type,\n"
        "    find_layers_by_selection,\n"
        "    flatten_block_of_weights,\n"
        "    get_exponents_and_other_4bits_fp8_e4m3,\n"
        "    get_luts_from_huffman_table,\n"
        "    get_nbit_codec,\n"
        "    locate_block_by_regex,\n"
        ")\n"),
    "scripts/inference_dfsyn.py:11":
        "from dfloat.run import DFloatDiffSynthModelFP8, get_dfloat_model_name_or_path\n",
}


@pytest.mark.parametrize("where", sorted(_IMPORTS))
def test_reference_import_lines_resolve(where):
    ns = {}
    exec(compile(_IMPORTS[where], where, "exec"), ns)
    for name, obj in ns.items():
        if name.startswith("__"):
            continue
        mod = getattr(obj, "__module__", "")
        assert mod.startswith("dfloat"), (name, mod)


def test_dfloat_run_exports_the_reference_names():
    import dfloat.run as run

    for name in ("DFloatModel", "_decode", "get_dfloat_model_name_or_path",
                 "load_and_replace_tensors", "load_and_replace_tensors_parallel",
                 "DFloatDiffSynthModelFP8"):
        assert name in run.__all__ and callable(getattr(run, name)), name


def _cut(patterns, names):
    return [n for n in names if any(re.fullmatch(p, n) for p in patterns)]


def test_patterns_cut_the_reference_blocks():
    from dfloat.const import get_default_no_split_pattern, get_fp8_pattern_dict

    llm = get_fp8_pattern_dict("Qwen3ForCausalLM")
    assert get_fp8_pattern_dict("LlamaForCausalLM") is llm
    names = ["model.embed_tokens", "model.layers.0", "model.layers.35", "model.layers.0.mlp",
             "model.layers.0.self_attn", "lm_head", "model.norm"]
    assert _cut(llm["fp8"], names) == ["model.layers.0", "model.layers.35"]
    assert _cut(llm["bf16"], names) == ["model.embed_tokens", "lm_head"]

    moe = get_fp8_pattern_dict("Qwen3MoeForCausalLM")
    names = ["model.layers.3", "model.layers.3.self_attn", "model.layers.3.mlp",
             "model.layers.3.mlp.gate", "model.layers.3.mlp.experts.127",
             "model.layers.3.mlp.experts.127.down_proj"]
    assert _cut(moe["fp8"], names) == ["model.layers.3.self_attn",
                                       "model.layers.3.mlp.experts.127"]

    # DeepSeek-V3: layers 0-2 whole; from layer 3 on, attention, shared
    # experts and each routed expert, never the router
    ds = get_fp8_pattern_dict("DeepseekV3ForCausalLM")
    names = ["model.layers.0", "model.layers.2", "model.layers.3", "model.layers.3.self_attn",
             "model.layers.2.self_attn", "model.layers.20.mlp.shared_experts",
             "model.layers.29.mlp.experts.255", "model.layers.29.mlp.gate",
             "model.layers.1.mlp.experts.0", "model.layers.10.self_attn"]
    assert _cut(ds["fp8"], names) == [
        "model.layers.0", "model.layers.2", "model.layers.3.self_attn",
        "model.layers.20.mlp.shared_experts", "model.layers.29.mlp.experts.255",
        "model.layers.10.self_attn"]

    flux = get_fp8_pattern_dict("FluxImagePipeline")
    assert isinstance(flux["fp8"], dict) and flux["bf16"] == []
    assert sorted(flux["fp8"][r"dit\.blocks\.\d+"]) == sorted(
        ["attn.a_to_out", "attn.a_to_qkv", "attn.b_to_out", "attn.b_to_qkv",
         "ff_a.0", "ff_a.2", "ff_b.0", "ff_b.2"])
    assert _cut(flux["fp8"], ["dit.blocks.18", "dit.single_blocks.37", "dit.blocks.1.attn",
                              "text_encoder_2.encoder.block.23"]) == [
        "dit.blocks.18", "dit.single_blocks.37", "text_encoder_2.encoder.block.23"]
    wan = get_fp8_pattern_dict("WanVideoPipeline")
    assert _cut(wan["fp8"], ["dit.blocks.3", "dit2.blocks.3", "text_encoder.blocks.1",
                             "vae.blocks.1"]) == ["dit.blocks.3", "dit2.blocks.3",
                                                  "text_encoder.blocks.1"]
    qi = get_fp8_pattern_dict("QwenImagePipeline")
    assert _cut(qi["fp8"], ["text_encoder.lm_head", "text_encoder.model.visual",
                            "dit.transformer_blocks.59", "text_encoder.model.language_model.layers.2",
                            "vae.decoder"]) == [
        "text_encoder.lm_head", "text_encoder.model.visual", "dit.transformer_blocks.59",
        "text_encoder.model.language_model.layers.2"]

    # a device placement keeps each compressed block whole
    assert _cut(get_default_no_split_pattern("Qwen3MoeForCausalLM"),
                ["model.layers.7", "model.layers.7.mlp.experts.3", "lm_head"]) == [
        "model.layers.7", "lm_head"]
    assert get_default_no_split_pattern("QwenImagePipeline") == qi["fp8"]
    with pytest.raises(ValueError, match="not supported"):
        get_fp8_pattern_dict("GPT2LMHeadModel")


def test_report_model_size_counts_pattern_bytes():
    from dfloat.utils import param_to_bytes, report_model_size

    m = torch.nn.Module()
    m.a = torch.nn.Linear(4, 8, bias=False)                       # 32 fp32 = 128 B
    m.b = torch.nn.Linear(4, 2, bias=True).to(torch.bfloat16)     # 10 bf16 = 20 B
    m.register_buffer("codes", torch.zeros(6, dtype=torch.uint8))  # 6 B
    gib = 1024 ** 3
    inc, exc, tot = report_model_size(m, [r"^a\."])
    assert (inc * gib, exc * gib, tot * gib) == (128, 26, 154)
    inc, exc, tot = report_model_size(m, {r"^b\.": ["bias"]})
    assert (round(inc * gib), round(exc * gib)) == (4, 150)
    assert report_model_size(m, None)[0] * gib == 154
    with pytest.raises(ValueError):
        param_to_bytes(torch.zeros(2, dtype=torch.complex64))


def _flux_cfg():
    from ecf8_amd.dit import FluxConfig

    return FluxConfig(hidden=256, heads=2, mlp=512, double=2, single=3, txt_dim=128,
                      pooled_dim=128)


def test_diffsynth_layout_round_trip(tmp_path):
    from dfloat.compress import compress_model
    from dfloat.const import get_fp8_pattern_dict
    from dfloat.run import DFloatDiffSynthModelFP8
    from ecf8_amd.dit import DOUBLE_LINEARS, SINGLE_LINEARS, random_pipeline

    pipe, _ = random_pipeline(_flux_cfg(), "cpu", seed=3)
    groups = (("dit.blocks", DOUBLE_LINEARS, 2), ("dit.single_blocks", SINGLE_LINEARS, 3))
    originals = {f"{p}.{i}": {n: pipe.get_submodule(f"{p}.{i}.{n}").weight.detach()
                              .view(torch.uint8).clone() for n in names}
                 for p, names, count in groups for i in range(count)}
    d = str(tmp_path / "flux-DF6.5")
    fp8 = get_fp8_pattern_dict("FluxImagePipeline")["fp8"]
    pattern = compress_model(pipe, fp8, d)

    # one file per block with the block module's state under its full names
    files = sorted(f for f in os.listdir(d) if f.endswith(".safetensors"))
    assert files == sorted(f"{b}.safetensors" for b in originals)
    from safetensors.torch import load_file

    stored = load_file(os.path.join(d, "dit.blocks.1.safetensors"))
    assert {"dit.blocks.1.luts", "dit.blocks.1.encoded", "dit.blocks.1.split_positions"} <= set(stored)
    assert all(k.startswith("dit.blocks.1.") for k in stored)
    assert not any(k.endswith("a_to_qkv.weight") for k in stored)
    with open(os.path.join(d, "dfloat_config.json")) as f:
        assert json.load(f) == {"version": "0.2.0", "threads_per_block": 512,
                                "bytes_per_thread": 8}
    assert pattern["fp8"][r"dit\.blocks\.\d+"] == list(DOUBLE_LINEARS)
    assert pattern["fp8"][r"dit\.single_blocks\.\d+"] == list(SINGLE_LINEARS)
    assert pattern["fp8"][r"text_encoder_2\.encoder\.block\.\d+"] is None  # no text encoder here

    fresh, _ = random_pipeline(_flux_cfg(), "cpu", seed=3)
    loaded = DFloatDiffSynthModelFP8.from_pretrained(d, "local/flux-DF6.5", fresh, device="cpu")
    assert loaded is fresh
    with open(os.path.join(d, "model_size.csv")) as f:
        assert f.readline().strip() == "fp8_blocks,rest,total"
    for block, orig in originals.items():
        blk = loaded.get_submodule(block)
        assert len(blk._forward_pre_hooks) == 1
        names = list(orig)
        assert [type(m).__name__ for m in blk.weight_injection_modules] == ["_Lin"] * len(names)
        flat = oc.decode(blk.luts.numpy(), blk.encoded.numpy(), blk.packed_other_4bits.numpy(),
                         blk.output_positions.numpy(), blk.gaps.numpy())
        for n, part in zip(names, np.split(flat, blk.split_positions)):
            assert np.array_equal(part, orig[n].numpy().reshape(-1)), (block, n)
            assert "weight" not in blk.get_submodule(n)._parameters


def test_diffsynth_pipeline_by_hub_name_is_refused(tmp_path):
    from dfloat.run import DFloatDiffSynthModelFP8

    (tmp_path / "x").mkdir()
    with pytest.raises((ImportError, ValueError)):
        DFloatDiffSynthModelFP8.from_pretrained(str(tmp_path / "x"), "DFloat11/FLUX.1-dev-DF6.5",
                                                "black-forest-labs/FLUX.1-dev", device="cpu")
    with pytest.raises(FileNotFoundError):
        DFloatDiffSynthModelFP8.from_pretrained(str(tmp_path / "missing"), "x", object())
