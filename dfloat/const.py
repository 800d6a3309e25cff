"""Which blocks of each supported model are compressed (dfloat/const.py:1-165).

A *block* is one module whose FP8 Linears are flattened into one compressed
stream and decoded by one forward-pre-hook.  Each family lists:

* ``fp8``  either a list of block regexes (every FP8 Linear under a matching
           block is compressed), or {block regex: [Linear paths inside the
           block]} for pipelines whose blocks also hold layers that stay;
* ``bf16`` regexes of modules kept uncompressed (written to pattern_dict.json);
* the model classes that use the family, and the regexes of modules a
  multi-GPU placement must not split (one block = one device, because the
  hook decodes into that device's buffer).

The regexes are part of the checkpoint contract: pattern_dict.json stores
them and the loader matches module names against them, so they are the
reference's strings, unchanged.
"""

from __future__ import annotations

_LAYER = r"model\.layers\.\d+"
_EMBED_HEAD = [r"model\.embed_tokens", r"lm_head"]

# layers 0-2 of DeepSeek-V3 are dense; later layers are cut per expert
_DSV3_LATER = r"model\.layers\.(?![0-2](?:[^0-9]|$))\d+"

_WAN_DIT_LINEARS = sorted([
    "cross_attn.k", "cross_attn.o", "cross_attn.q", "cross_attn.v", "ffn.0", "ffn.2",
    "self_attn.k", "self_attn.o", "self_attn.q", "self_attn.v",
])

_FAMILIES = {
    "llm": dict(
        classes=["Qwen3ForCausalLM", "LlamaForCausalLM"],
        fp8=[_LAYER],
        bf16=_EMBED_HEAD,
        no_split=[r"model\.embed_tokens", _LAYER, r"lm_head"],
    ),
    "deepseekv3": dict(
        classes=["DeepseekV3ForCausalLM"],
        fp8=[
            r"model\.layers\.[0-2]",
            _DSV3_LATER + r"\.self_attn",
            _DSV3_LATER + r"\.mlp\.shared_experts",
            _DSV3_LATER + r"\.mlp\.experts\.\d+",
        ],
        bf16=_EMBED_HEAD,
        no_split=[r"model\.embed_tokens", _LAYER, r"lm_head"],
    ),
    "qwen3moe": dict(
        classes=["Qwen3MoeForCausalLM"],
        fp8=[_LAYER + r"\.self_attn", _LAYER + r"\.mlp\.experts\.\d+"],
        bf16=_EMBED_HEAD,
        no_split=[r"model\.embed_tokens", _LAYER, r"lm_head"],
    ),
    "diffsynth-flux-fp8": dict(
        classes=["FluxImagePipeline"],
        fp8={
            r"text_encoder_2\.encoder\.block\.\d+": [
                f"layer.0.SelfAttention.{p}" for p in ("k", "o", "q", "v")],
            r"dit\.blocks\.\d+": [
                "attn.a_to_out", "attn.a_to_qkv", "attn.b_to_out", "attn.b_to_qkv",
                "ff_a.0", "ff_a.2", "ff_b.0", "ff_b.2"],
            r"dit\.single_blocks\.\d+": ["norm.linear", "proj_out", "to_qkv_mlp"],
        },
        bf16=[],
        no_split=[r"text_encoder_2\.encoder\.block\.\d+", r"dit\.blocks\.\d+",
                  r"dit\.single_blocks\.\d+"],
    ),
    "diffsynth-wanvideo-fp8": dict(
        classes=["WanVideoPipeline"],
        fp8={
            r"text_encoder\.blocks\.\d+": sorted([
                "attn.k", "attn.o", "attn.q", "attn.v", "ffn.fc1", "ffn.fc2", "ffn.gate.0"]),
            r"dit\.blocks\.\d+": list(_WAN_DIT_LINEARS),
            r"dit2\.blocks\.\d+": list(_WAN_DIT_LINEARS),
        },
        bf16=[],
        no_split=[r"text_encoder\.blocks\.\d+", r"dit\.blocks\.\d+", r"dit2\.blocks\.\d+"],
    ),
    "diffsynth-qwenimage-fp8": dict(
        classes=["QwenImagePipeline"],
        fp8=[
            r"text_encoder\.lm_head",
            r"text_encoder\.model\.visual",
            r"text_encoder\.model\.language_model\.layers\.\d+",
            r"dit\.transformer_blocks\.\d+",
        ],
        bf16=[],
        no_split=None,  # same as its fp8 blocks
    ),
}

FP8_PATTERN_DICT = {k: {"fp8": f["fp8"], "bf16": f["bf16"]} for k, f in _FAMILIES.items()}
MODEL_CLASS_MAP = {k: set(f["classes"]) for k, f in _FAMILIES.items()}
DEFAULT_NO_SPLIT_PATTERN = {
    k: list(f["no_split"] if f["no_split"] is not None else f["fp8"])
    for k, f in _FAMILIES.items()
}


def _family(model_class: str) -> str:
    for key, classes in MODEL_CLASS_MAP.items():
        if model_class in classes:
            return key
    raise ValueError(f"Model class {model_class} not supported")


def get_fp8_pattern_dict(model_class: str) -> dict:
    """{"fp8": ..., "bf16": ...} of the family ``model_class`` belongs to
    (dfloat/const.py:154-159); ValueError for an unknown class."""
    return FP8_PATTERN_DICT[_family(model_class)]


def get_default_no_split_pattern(model_class: str) -> list:
    """Regexes of the modules a device placement keeps whole
    (dfloat/const.py:162-165)."""
    return DEFAULT_NO_SPLIT_PATTERN[_family(model_class)]
