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
    vals, freqs = torch.unique(exps, return_counts=True)
    p = freqs / freqs.sum()
    entropy = float(-torch.sum(p * torch.log2(p)).item()) if freqs.numel() else 0.0
    counter = {int(v): int(f) for v, f in zip(vals.tolist(), freqs.tolist())}
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
    from .decode import decode

    dev = torch.device(device)
    moved = {k: tensors[k].to(dev) for k in ("luts", "encoded", "packed_other_4bits",
                                            "output_positions", "gaps")}
    out = decode(moved["luts"], moved["encoded"], moved["packed_other_4bits"],
                 moved["output_positions"], moved["gaps"],
                 threads_per_block=result["threads_per_block"],
                 bytes_per_thread=result["bytes_per_thread"])
    assert torch.equal(tensors["flat_weights"].view(torch.uint8), out.cpu().view(torch.uint8))


validate_gpu_decoding_fp8 = validate_cuda_decoding_fp8
