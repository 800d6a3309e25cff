"""Per-block compression pipeline and GPU round-trip check
(scripts/compress.py:70-270 without the hub model loading).

A compressed block is the dict of tensors the reference caches and registers
as buffers (scripts/compress.py:239-247, 607-612):
``luts`` u8[n_luts,256], ``encoded`` u8, ``packed_other_4bits`` u8[n/2],
``output_positions`` u8 view of u64[n_fb+1], ``gaps`` u8,
``split_positions`` int64, plus ``flat_weights`` e4m3fn in the cache file.
"""

from __future__ import annotations

import json
import os
import re

import torch

from .utils import (
    encode_exponents_for_cuda,
    flatten_block_of_weights,
    get_exponents_and_other_4bits_fp8_e4m3,
    get_luts_from_huffman_table,
    get_nbit_codec,
)

PACKAGE_FORMAT_VERSION = "0.2.0"  # dfloat_config["version"] (scripts/compress.py:67)


def compress_flat(flat_weights: torch.Tensor, bytes_per_thread: int = 8,
                  threads_per_block: int = 512) -> dict:
    """Compress one flattened e4m3fn block (scripts/compress.py:197-247):
    split, count exponents in ascending order, length-limited codebook,
    LUTs, bitstream.  Returns the tensors plus ``entropy`` and ``table``."""
    exps, packed = get_exponents_and_other_4bits_fp8_e4m3(flat_weights)
    # a 16-bin count is O(n); the reference's ascending-symbol counter order
    # (scripts/compress.py:205, 213-215) is kept by listing present symbols
    counts = torch.bincount(exps.reshape(-1), minlength=16)
    present = counts > 0
    freqs = counts[present]
    p = freqs.double() / freqs.sum()
    entropy = float(-torch.sum(p * torch.log2(p)).item()) if freqs.numel() else 0.0
    counter = {int(v): int(counts[v]) for v in torch.nonzero(present).reshape(-1).tolist()}
    codec, _, table = get_nbit_codec(counter, max_n_bits=16)
    luts = get_luts_from_huffman_table(table)
    encoded, gaps, op = encode_exponents_for_cuda(exps, codec, bytes_per_thread, threads_per_block)
    return {
        "flat_weights": flat_weights,
        "luts": luts,
        "encoded": encoded,
        "packed_other_4bits": packed.contiguous(),
        "output_positions": op.view(torch.uint8),
        "gaps": gaps,
        "entropy": entropy,
        "table": table,
    }


def process_fp8_block(block_item, info_dict):
    """Compress one block and cache it under ``save_path/cache`` as
    ``{block}.safetensors`` (tensor names as in scripts/compress.py:239-247)
    with JSON metadata ``{block}.json``; a block whose two files exist is not
    recompressed (resume, scripts/compress.py:163-186)."""
    from safetensors.torch import load_file, save_file

    block_name, layers = block_item
    cache_dir = os.path.join(info_dict["save_path"], "cache")
    os.makedirs(cache_dir, exist_ok=True)
    tensor_path = os.path.join(cache_dir, block_name + ".safetensors")
    meta_path = os.path.join(cache_dir, block_name + ".json")
    bpt = info_dict["bytes_per_thread"]
    tpb = info_dict["threads_per_block"]

    layer_names = []
    for name in layers:
        if not (name.startswith(block_name + ".") or name == block_name):
            raise Exception(f"Layer name mismatch: layer {name} block {block_name}")
        layer_names.append(name[len(block_name) + 1:])
    matched = next((r for r in info_dict["model_fp8_regex"] if re.fullmatch(r, block_name)), None)

    if os.path.exists(tensor_path) and os.path.exists(meta_path):
        with open(meta_path) as f:
            entropy = json.load(f)["entropy"]
    else:
        flat, split_positions = flatten_block_of_weights(layers, dtype=torch.float8_e4m3fn)
        res = compress_flat(flat, bpt, tpb)
        entropy = res["entropy"]
        save_file({
            "flat_weights": flat,
            "luts": res["luts"],
            "encoded": res["encoded"],
            "packed_other_4bits": res["packed_other_4bits"],
            "output_positions": res["output_positions"],
            "gaps": res["gaps"],
            "split_positions": split_positions,
        }, tensor_path)
        load_file(tensor_path)  # fail now, not at load time, on a bad write

    meta = {
        "block_name": block_name,
        "layer_names": layer_names,
        "matched_regex": matched,
        "layers_to_delete": list(layers),
        "threads_per_block": tpb,
        "bytes_per_thread": bpt,
        "block_save_path": tensor_path,
        "entropy": entropy,
    }
    with open(meta_path, "w") as f:
        json.dump(meta, f)
    return meta


def validate_cuda_decoding_fp8(result, tensors, device) -> None:
    """GPU round trip of one cached block against its original FP8 bytes,
    the reference's check (scripts/compress.py:70-126), through the HIP
    decoder.  Raises AssertionError on any differing byte."""
    from ecf8_amd.decode import decode

    dev = torch.device(device)
    moved = {k: tensors[k].to(dev) for k in ("luts", "encoded", "packed_other_4bits",
                                            "output_positions", "gaps")}
    out = decode(moved["luts"], moved["encoded"], moved["packed_other_4bits"],
                 moved["output_positions"], moved["gaps"],
                 threads_per_block=result["threads_per_block"],
                 bytes_per_thread=result["bytes_per_thread"])
    assert torch.equal(tensors["flat_weights"].view(torch.uint8), out.cpu().view(torch.uint8))


validate_gpu_decoding_fp8 = validate_cuda_decoding_fp8


def compressible_linear_types() -> tuple:
    """The module types whose e4m3fn ``weight`` a block contributes
    (scripts/compress.py:519-528): ``nn.Linear``, transformers' ``FP8Linear``
    (every quantized Linear of an HF FP8 checkpoint) and DiffSynth's
    ``AutoWrappedLinear``, each when importable.  Matching is by exact type,
    as the reference's finder does (dfloat/utils.py:165)."""
    types = [torch.nn.Linear]
    try:
        from transformers.integrations.finegrained_fp8 import FP8Linear
        types.append(FP8Linear)
    except ImportError:
        pass
    try:
        from diffsynth.core.vram.layers import AutoWrappedLinear
        types.append(AutoWrappedLinear)
    except ImportError:
        pass
    return tuple(types)


def fp8_layers_by_block(model, fp8_regex) -> dict:
    """{block name: {layer name: module}} of the FP8 layers to compress
    (scripts/compress.py:515-536): with a list of block regexes, every FP8
    layer of a ``compressible_linear_types`` type under each matching block;
    with a dict {regex: layer paths}, the selected layers of each matching
    block.  A matching block without a single FP8 layer raises ValueError:
    its checkpoint would be written as compressed while holding nothing
    compressed."""
    from .utils import (find_layers_by_data_type_and_layer_type, find_layers_by_selection,
                        locate_block_by_regex)

    out = {}
    if isinstance(fp8_regex, dict):
        for regex, selected in fp8_regex.items():
            for name, block in locate_block_by_regex(model, regex).items():
                out[name] = find_layers_by_selection(block, selected, name=name)
    else:
        layer_types = compressible_linear_types()
        for name, block in locate_block_by_regex(model, "|".join(fp8_regex)).items():
            out[name] = find_layers_by_data_type_and_layer_type(
                block, target_dtype=torch.float8_e4m3fn, layers=layer_types, name=name)
    empty = [k for k, v in out.items() if not v]
    if empty:
        raise ValueError(f"{len(empty)} block(s) matching the FP8 patterns hold no float8_e4m3fn "
                         f"layer of types {[t.__name__ for t in compressible_linear_types()]}: "
                         f"{empty[:4]}")
    return out


def _layout(model, fp8_regex, layout: str) -> str:
    if layout != "auto":
        if layout not in ("hf", "diffsynth", "full"):
            raise ValueError(f"unknown checkpoint layout {layout!r}")
        return layout
    if hasattr(model, "save_pretrained") and hasattr(model, "config"):
        return "hf"
    return "diffsynth" if isinstance(fp8_regex, dict) else "full"


def compress_model(model, fp8_regex, save_path: str, threads_per_block: int = 512,
                   bytes_per_thread: int = 8, bf16_regex=(), validate_device=None,
                   n_workers: int = 1, layout: str = "auto", tokenizer=None) -> dict:
    """Compress every FP8 block of a local model and save the checkpoint the
    way scripts/compress.py:490-680 does.

    Each block's layers are removed and its compressed tensors registered as
    buffers on the block module (:583-612); ``validate_device`` runs the
    GPU round trip of every block first (:571-585); the block regexes and
    their Linear names go to ``pattern_dict.json`` ({"fp8": {regex: layer
    names}, "bf16": {regex: []}}, :634-680) and each block's entropy to
    ``entropy.csv``.  The checkpoint itself, by ``layout``:

    * ``"hf"`` (default for a transformers model): ``model.config`` gets
      ``dfloat_config`` = {version, threads_per_block, bytes_per_thread} and
      the model is written by ``save_pretrained``; ``tokenizer``, if given,
      is saved beside it (:668-677).  ``DFloatModel.from_pretrained`` reads
      this directory;
    * ``"diffsynth"`` (default for a {regex: layer paths} pattern, the
      DiffSynth pipelines): one ``<block>.safetensors`` per block with the
      block module's state dict under its full names (:614-624), plus
      ``dfloat_config.json``; the pipeline's other weights stay with the
      original model.  ``DFloatDiffSynthModelFP8.from_pretrained`` reads it;
    * ``"full"`` (default for any other module): the whole state dict in
      ``model.safetensors`` plus ``dfloat_config.json``, for modules that
      have neither a Hugging Face config nor a pipeline of their own.

    ``n_workers`` > 1 compresses the blocks in a thread pool, as the
    reference's pool does (scripts/compress.py:320-361; the encoder and the
    tensor work release the interpreter lock); 1 is the reference's
    --sequential path.  Registration, validation and saving follow in block
    order either way.  Returns the pattern dict."""
    import operator

    from safetensors.torch import load_file, save_file

    layout = _layout(model, fp8_regex, layout)
    os.makedirs(save_path, exist_ok=True)
    regexes = list(fp8_regex.keys()) if isinstance(fp8_regex, dict) else list(fp8_regex)
    regex_dict = {r: None for r in regexes}
    info = {"save_path": save_path, "model_fp8_regex": regexes,
            "bytes_per_thread": bytes_per_thread, "threads_per_block": threads_per_block}
    items = list(fp8_layers_by_block(model, fp8_regex).items())
    if not items:
        raise ValueError(f"no module of the model matches the FP8 block patterns {regexes}")
    if n_workers > 1 and len(items) > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=min(n_workers, len(items))) as ex:
            results = list(ex.map(lambda item: process_fp8_block(item, info), items))
    else:
        results = [process_fp8_block(item, info) for item in items]
    entropies = {}
    for (block_name, _layers), result in zip(items, results):
        tensors = load_file(result["block_save_path"])
        if validate_device is not None:
            validate_cuda_decoding_fp8(result, tensors, validate_device)
        entropies[block_name] = result["entropy"]
        block = operator.attrgetter(block_name)(model)
        for layer_name in result["layers_to_delete"]:
            if layer_name == block_name:
                delattr(block, "weight")
            else:
                parent_name, attr = layer_name.rsplit(".", 1)
                delattr(operator.attrgetter(parent_name)(model), attr)
        for key in ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps",
                    "split_positions"):
            block.register_buffer(key, tensors[key])
        if layout == "diffsynth":
            state = {f"{block_name}.{k}": v.contiguous() for k, v in block.state_dict().items()}
            save_file(state, os.path.join(save_path, block_name + ".safetensors"))
        matched = result["matched_regex"]
        if matched:
            if regex_dict[matched] is None:
                regex_dict[matched] = result["layer_names"]
            elif regex_dict[matched] != result["layer_names"]:
                raise ValueError(f"{block_name}: layers {result['layer_names']} differ from "
                                 f"{regex_dict[matched]} of the other blocks of {matched}")
    with open(os.path.join(save_path, "entropy.csv"), "w") as f:
        f.write("block_name,entropy\n")
        for name in sorted(entropies):
            f.write(f"{name},{entropies[name]}\n")
    dfloat_config = {"version": PACKAGE_FORMAT_VERSION, "threads_per_block": threads_per_block,
                     "bytes_per_thread": bytes_per_thread}
    if layout == "hf":
        model.config.dfloat_config = dfloat_config
        model.save_pretrained(save_path)
        if tokenizer is not None:
            tokenizer.save_pretrained(save_path)
    else:
        if layout == "full":
            state = {k: v.contiguous() for k, v in model.state_dict().items()}
            save_file(state, os.path.join(save_path, "model.safetensors"))
        with open(os.path.join(save_path, "dfloat_config.json"), "w") as f:
            json.dump(dfloat_config, f, indent=4)
    pattern_dict = {"fp8": regex_dict, "bf16": {r: [] for r in bf16_regex}}
    with open(os.path.join(save_path, "pattern_dict.json"), "w") as f:
        json.dump(pattern_dict, f, indent=4)
    return pattern_dict
