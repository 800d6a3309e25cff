"""Runtime of the reference's ``dfloat.run`` (dfloat/run/run.py).

* ``_decode``          callable with the cp.RawKernel call form the reference
                       uses (grid=, block=, shared_mem=, args=[...]);
* ``TensorManager``    one grow-only e4m3fn decode buffer per device;
* ``get_hook``         forward-pre-hook: decode the module's compressed block
                       into the buffer and inject ``.weight`` views;
* ``load_and_replace_tensors[_parallel]`` / ``_process_compressed_tensor``
                       register compressed buffers + hooks from safetensors;
* ``DFloatModel``, ``DFloatDiffSynthModelFP8``
                       loaders of compressed checkpoints from local
                       directories (no hub download).

Decode launches go on torch's current stream of the module's device through
the C ABI of libecf8 (``ecf8_amd.decode``), so decode and the consuming GEMM
are ordered without any cross-runtime synchronisation.
"""

from __future__ import annotations

import json
import os
import re
from sys import stderr
from typing import Dict, Optional, Union

import torch
import torch.nn as nn

from ecf8_amd import decode as _dev
from ecf8_amd._lib import ECF8_TABLE_ANY, ECF8_TABLE_CACHE_BYTES, ECF8Error, check, lib
from ecf8_amd.hf_fp8 import bind_fp8_linears

__all__ = [
    "DFloatModel",
    "_decode",
    "get_dfloat_model_name_or_path",
    "load_and_replace_tensors",
    "load_and_replace_tensors_parallel",
    "load_compressed_model",
    "DFloatDiffSynthModelFP8",
    "TensorManager",
    "get_hook",
    "get_no_split_classes",
]


class _DecodeLauncher:
    """Call-compatible stand-in for ``_decode = cp.RawKernel(decode.cu,
    "decode")`` (dfloat/run/run.py:24-33).  ``args`` are the reference
    kernel's: luts, encoded, packed_other_4bits, output_positions, gaps,
    outputs (device addresses), n_luts, n_bytes, n_elements
    (decode.cu:16-26).  Like the reference's launch it is asynchronous on the
    current stream.

    The decode reads a derived table of the LUTs.  Each (device, stream, LUT
    address, n_luts) keeps one table cache (``ecf8_build_table_cached``):
    before every decode a one-workgroup kernel compares the LUT bytes with
    the ones the cached table was built from and rebuilds it only if they
    changed, so a LUT buffer rewritten between calls is always decoded with
    its current contents, and an unchanged one costs a compare instead of a
    rebuild.  The decode reads the table's kind on the device.  Nothing
    returns to the host, so calls can be captured in a HIP graph.  At most
    ``max_cached`` caches are kept (least recently used dropped first;
    ECF8_TABLE_CACHE_BYTES each); ``clear()`` drops them all."""

    max_cached = 512

    def __init__(self):
        from collections import OrderedDict

        self._caches = OrderedDict()

    def clear(self):
        self._caches.clear()

    def _table_cache(self, dev: int, st, luts: int, n_luts: int) -> torch.Tensor:
        key = (dev, st.cuda_stream, luts, n_luts)
        cache = self._caches.get(key)
        if cache is None:
            with torch.cuda.stream(st):
                # zero-filled: never matches a LUT stack (n_luts >= 2)
                cache = torch.zeros(ECF8_TABLE_CACHE_BYTES // 8, dtype=torch.int64,
                                    device=torch.device("cuda", dev))
            self._caches[key] = cache
            while len(self._caches) > self.max_cached:
                self._caches.popitem(last=False)
        else:
            self._caches.move_to_end(key)
        return cache

    def __call__(self, grid, block, args, shared_mem: int = 0, stream=None):
        luts, encoded, packed, op, gaps, outputs, n_luts, n_bytes, n_elements = args
        tpb = int(block[0] if isinstance(block, (tuple, list)) else block)
        # the reference's shared_mem = tpb*4 + 4 + largest block (run.py:268-270)
        max_block = max(0, int(shared_mem) - tpb * 4 - 4)
        nblk = int(grid[0] if isinstance(grid, (tuple, list)) else grid)
        bpt = 8
        if nblk != _dev.n_format_blocks(n_bytes, tpb, bpt):
            raise ECF8Error(f"grid {nblk} does not cover {n_bytes} bytes with {tpb} threads")
        dev = torch.cuda.current_device()
        st = torch.cuda.current_stream(dev) if stream is None else stream
        cache = self._table_cache(dev, st, int(luts), int(n_luts))
        s = st.cuda_stream
        L = lib()
        check(L.ecf8_build_table_cached(int(luts), int(n_luts), ECF8_TABLE_ANY, cache.data_ptr(),
                                        s), "ecf8_build_table_cached")
        check(L.ecf8_decode(int(luts), int(encoded), int(packed), int(op), int(gaps), int(outputs),
                            int(n_luts), int(n_bytes), int(n_elements), max_block, 0,
                            cache.data_ptr(), ECF8_TABLE_ANY, tpb, bpt, s), "ecf8_decode")


_decode = _DecodeLauncher()


def _device_key(device) -> torch.device:
    """``device`` with its index filled in ("cuda" -> "cuda:<current>"), so
    one device never holds two decode buffers."""
    d = torch.device(device)
    if d.type == "cuda" and d.index is None:
        d = torch.device("cuda", torch.cuda.current_device())
    return d


class TensorManager:
    """The decode buffer of each device, shared by every compressed block on
    it (the reference keeps one per device, dfloat/run/run.py:36-81).

    ``get_tensor`` hands out the first ``n_elements`` of the device's buffer.
    The buffer only grows: when a block needs more (or another dtype), the
    old buffer is released before the larger one is taken, so the two never
    hold memory at once.  Blocks decode one after another on a device, so
    sharing the buffer is safe; a caller that keeps a view past the next
    decode on that device sees the next block's weights."""

    _tensors: Dict[torch.device, torch.Tensor] = {}

    @classmethod
    def get_tensor(cls, device, n_elements: int, dtype=torch.float8_e4m3fn) -> torch.Tensor:
        key = _device_key(device)
        buf = cls._tensors.get(key)
        if buf is not None and buf.numel() >= n_elements and buf.dtype == dtype:
            return buf[:n_elements]
        if buf is not None:
            del cls._tensors[key], buf
            torch.cuda.empty_cache()
        buf = torch.empty(n_elements, dtype=dtype, device=key)
        cls._tensors[key] = buf
        print(f"[dfloat] decode buffer on {key}: {n_elements} elements of {dtype}", file=stderr)
        return buf

    @classmethod
    def clear_device(cls, device=None):
        """Release the buffer of ``device``, or of every device."""
        if device is None:
            cls._tensors.clear()
        else:
            cls._tensors.pop(_device_key(device), None)
        torch.cuda.empty_cache()


def _module_state(module: nn.Module):
    """Per-module decode state, derived once on the module's device and
    rebuilt if the buffers move: the derived decode table, the largest
    format-block (the quantity behind the reference's shared_mem_size) and
    the shortest code length, which size the kernel's LDS."""
    luts = module.luts
    key = (luts.device, luts.data_ptr(), module.output_positions.data_ptr())
    cached = module.__dict__.get("_ecf8_state")
    if cached is None or cached[0] != key:
        table = _dev.build_table(luts.contiguous())
        tpb = module.__dict__.get("_ecf8_tpb", 512)
        if hasattr(module, "shared_mem_size"):
            max_block = max(0, int(module.shared_mem_size) - tpb * 4 - 4)
        else:
            max_block = _dev.largest_block(module.output_positions)
        cached = (key, table, max_block, _dev.min_code_bits(luts))
        module.__dict__["_ecf8_state"] = cached
    return cached[1], cached[2], cached[3]


def _inject(module: nn.Module, reconstructed: torch.Tensor) -> None:
    """dfloat/run/run.py:121-153: a Linear/Embedding gets a 2-D view of the
    whole buffer; any other module's ``weight_injection_modules`` get views
    of ``tensor_split(reconstructed, split_positions)`` in order."""
    if isinstance(module, nn.Linear):
        module.weight = reconstructed.view(module.out_features, module.in_features)
    elif isinstance(module, nn.Embedding):
        module.weight = reconstructed.view(module.num_embeddings, module.embedding_dim)
    else:
        parts = torch.tensor_split(reconstructed, module.split_positions)
        for sub, w in zip(module.weight_injection_modules, parts):
            if isinstance(sub, nn.Embedding):
                sub.weight = w.view(sub.num_embeddings, sub.embedding_dim)
            elif isinstance(sub, nn.Module) and hasattr(sub, "out_features"):
                sub.weight = w.view(sub.out_features, sub.in_features)
            else:
                raise ValueError(f"Unsupported module type: {type(sub)}")


def _injected(module: nn.Module):
    """(module, weight tensor) pairs _inject set on this block."""
    targets = [module] if isinstance(module, (nn.Linear, nn.Embedding)) else \
        list(module.weight_injection_modules)
    return [(t, t.__dict__.get("weight")) for t in targets]


def get_hook(threads_per_block: int, bytes_per_thread: int):
    """Forward-pre-hook factory (dfloat/run/run.py:84-155): decode the
    module's compressed block on its device's current stream into the shared
    TensorManager buffer, then inject the weight views.

    The first call checks every buffer (decode_into) and injects the views;
    it keeps the packed launch arguments and the injected views, keyed by
    the buffers' and the output's addresses.  A later call with the same
    key makes that one launch, and injects again only if a view was
    replaced in between: the views of an unchanged buffer are the same
    views, and a block's host time here is GPU idle time in an eager
    forward that issues thousands of small kernels.  Like the derived table,
    the kept arguments assume a block's compressed buffers are not rewritten
    in place: new weights loaded into the same storage need the module's
    ``_ecf8_state`` and ``_ecf8_launch`` entries dropped first."""

    def decode_hook(module, _):
        n_elements = module.packed_other_4bits.numel() * 2
        device = module.encoded.device
        reconstructed = TensorManager.get_tensor(device, n_elements)
        key = (reconstructed.data_ptr(), module.luts.data_ptr(), module.encoded.data_ptr(),
               module.packed_other_4bits.data_ptr(), module.output_positions.data_ptr(),
               module.gaps.data_ptr(), n_elements)
        fast = module.__dict__.get("_ecf8_launch")
        if fast is not None and fast[0] == key:
            _, fn, args, views, _table = fast
            rc = fn(*args, torch.cuda.current_stream(device).cuda_stream)
            if rc:
                check(rc, "ecf8_decode")
            if any(t.__dict__.get("weight") is not v for t, v in views):
                _inject(module, reconstructed)
                module.__dict__["_ecf8_launch"] = fast[:3] + (_injected(module), fast[4])
            return
        module.__dict__["_ecf8_tpb"] = threads_per_block
        table, max_block, min_bits = _module_state(module)
        _dev.decode_into(reconstructed, module.luts, module.encoded, module.packed_other_4bits,
                         module.output_positions, module.gaps, table=table,
                         threads_per_block=threads_per_block, bytes_per_thread=bytes_per_thread,
                         max_block_elements=max_block, min_code_bits=min_bits)
        _inject(module, reconstructed)
        args = (module.luts.data_ptr(), module.encoded.data_ptr(),
                module.packed_other_4bits.data_ptr(), module.output_positions.data_ptr(),
                module.gaps.data_ptr(), reconstructed.data_ptr(), _dev._n_luts(module.luts),
                module.encoded.numel(), n_elements, int(max_block), int(min_bits),
                table.data.data_ptr(), int(table.kind), threads_per_block, bytes_per_thread)
        module.__dict__["_ecf8_launch"] = (key, lib().ecf8_decode, args, _injected(module), table)

    return decode_hook


def _shared_mem_size(module, threads_per_block: int) -> int:
    op = module.output_positions.view(torch.uint64).cpu().numpy().astype("int64")
    per_block = op[1:] - op[:-1]
    longest = int(per_block.max()) if per_block.size else 0
    return threads_per_block * 4 + 4 + longest


def _process_compressed_tensor(module, attr_name, tensor_value, tensor_name, pattern_dict,
                               threads_per_block, bytes_per_thread):
    """Attach one tensor of a compressed block to its module, as the
    reference's loader does (dfloat/run/run.py:406-458).

    ``split_positions`` is kept as a list of ints; every other tensor becomes
    a buffer.  Two tensors trigger more: ``output_positions`` fixes the
    block's ``shared_mem_size``, and ``encoded`` -- the block itself -- gets
    the decode hook and gives up the dense weights it replaces
    (``_take_dense_weights``)."""
    if attr_name == "split_positions":
        module.split_positions = [int(v) for v in tensor_value.tolist()]
        return
    module.register_buffer(attr_name, tensor_value)
    if attr_name == "output_positions":
        module.shared_mem_size = _shared_mem_size(module, threads_per_block)
    elif attr_name == "encoded":
        module.register_forward_pre_hook(get_hook(threads_per_block, bytes_per_thread))
        _take_dense_weights(module, tensor_name.rpartition(".")[0], pattern_dict)


def _take_dense_weights(module, module_path: str, pattern_dict: dict) -> None:
    """Drop the dense weights a compressed block replaces.  The first
    pattern of ``pattern_dict`` that matches the block's path decides: a
    block that is itself a Linear or Embedding loses its own ``weight``;
    any other block loses the weights of the layers the pattern lists, and
    those layers, in that order, become its ``weight_injection_modules``
    (the hook's views of the decoded block go to them)."""
    layer_paths = next((paths for pattern, paths in pattern_dict.items()
                        if re.fullmatch(pattern, module_path)), None)
    if layer_paths is None:
        return
    if isinstance(module, (nn.Linear, nn.Embedding)):
        delattr(module, "weight")
        return
    targets = []
    for path in layer_paths:
        target = module.get_submodule(path)
        if not hasattr(target, "weight"):
            raise ValueError(f"{module_path}.{path} has no weight for the decoded block to replace")
        delattr(target, "weight")
        targets.append(target)
    module.weight_injection_modules = targets


def _process_file(model, path, pattern_dict, tpb, bpt, state_names, params, bufs, cache):
    from safetensors.torch import load_file

    loaded = load_file(path)
    for name, value in loaded.items():
        if name in state_names:
            target = params.get(name)
            if target is None:
                target = bufs[name]
            if target.shape == value.shape:
                target.data = value
            else:
                print(f"Shape mismatch for {name}: model {target.shape} vs loaded {value.shape}",
                      file=stderr)
            continue
        parts = name.split(".")
        mpath = ".".join(parts[:-1])
        module = cache.get(mpath)
        if module is None:
            module = model
            for p in parts[:-1]:
                if not hasattr(module, p):
                    print(f"Cannot find module path for {name}", file=stderr)
                    module = None
                    break
                module = getattr(module, p)
            if module is None:
                continue
            cache[mpath] = module
        _process_compressed_tensor(module, parts[-1], value, name, pattern_dict, tpb, bpt)
    return len(loaded)


def validate_compressed_modules(model, threads_per_block: int = 512, bytes_per_thread: int = 8):
    """Run the host format validator over every hooked module (buffers must
    still be reachable); raises ECF8Error on the first malformed block."""
    count = 0
    for name, m in model.named_modules():
        if all(hasattr(m, a) for a in ("luts", "encoded", "packed_other_4bits",
                                        "output_positions", "gaps")):
            try:
                _dev.validate_format(m.luts, m.encoded.numel(), m.packed_other_4bits.numel(),
                                     m.output_positions, m.gaps.numel(), threads_per_block,
                                     bytes_per_thread)
            except ECF8Error as e:
                raise ECF8Error(f"{name}: {e}") from None
            count += 1
    return count


def load_and_replace_tensors(model, directory_path, dfloat_config):
    """Sequential loader (dfloat/run/run.py:158-275)."""
    tpb = dfloat_config["threads_per_block"]
    bpt = dfloat_config["bytes_per_thread"]
    pattern_dict = dfloat_config["pattern_dict"]["fp8"]
    files = sorted(f for f in os.listdir(directory_path) if f.endswith(".safetensors"))
    state_names = set(model.state_dict().keys())
    params = dict(model.named_parameters())
    bufs = dict(model.named_buffers())
    cache = {}
    for f in files:
        _process_file(model, os.path.join(directory_path, f), pattern_dict, tpb, bpt, state_names,
                      params, bufs, cache)
    validate_compressed_modules(model, tpb, bpt)
    return model


def load_and_replace_tensors_parallel(model, directory_path, dfloat_config):
    """Thread-pooled loader over the safetensors files
    (dfloat/run/run.py:278-403).  Unlike the reference, a failing file
    raises instead of being counted as 0 tensors."""
    from concurrent.futures import ThreadPoolExecutor

    tpb = dfloat_config["threads_per_block"]
    bpt = dfloat_config["bytes_per_thread"]
    pattern_dict = dfloat_config["pattern_dict"]["fp8"]
    files = sorted(f for f in os.listdir(directory_path) if f.endswith(".safetensors"))
    state_names = set(model.state_dict().keys())
    params = dict(model.named_parameters())
    bufs = dict(model.named_buffers())
    cache = {}
    workers = max(1, min(8, len(files), os.cpu_count() or 4))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(_process_file, model, os.path.join(directory_path, f), pattern_dict,
                          tpb, bpt, state_names, params, bufs, cache) for f in files]
        total = sum(f.result() for f in futs)
    print(f"Processed {total} tensors from {len(files)} files", file=stderr)
    validate_compressed_modules(model, tpb, bpt)
    return model


def load_compressed_model(model, dfloat_dir: str, parallel: bool = False):
    """Load a compressed checkpoint directory into ``model`` (an instance of
    the original architecture): dfloat_config.json (or config.json's
    ``dfloat_config``) and pattern_dict.json as DFloatDiffSynthModelFP8 and
    DFloatModel read them (dfloat/run/run.py:510-522, 569-729), then the
    loader registers every block's buffers and decode hook."""
    cfg_path = os.path.join(dfloat_dir, "dfloat_config.json")
    if os.path.exists(cfg_path):
        with open(cfg_path) as f:
            dfloat_config = json.load(f)
    else:
        with open(os.path.join(dfloat_dir, "config.json")) as f:
            dfloat_config = dict(json.load(f)["dfloat_config"])
    with open(os.path.join(dfloat_dir, "pattern_dict.json")) as f:
        dfloat_config["pattern_dict"] = json.load(f)
    loader = load_and_replace_tensors_parallel if parallel else load_and_replace_tensors
    return loader(model, dfloat_dir, dfloat_config)


def get_dfloat_model_name_or_path(repo_id: str, dfloat_dir: str = "../dfloat-models"):
    """Local directory and hub id of a compressed model
    (dfloat/run/run.py:473-480)."""
    parts = repo_id.split("/")
    parts[0] = "DFloat11"
    dfloat_model_id = "/".join(parts) + "-DF6.5"
    dfloat_repo_id = os.path.join(dfloat_dir, "models--" + "--".join(parts) + "-DF6.5")
    return dfloat_repo_id, dfloat_model_id


def get_no_split_classes(model, patterns) -> list:
    """Class names of the modules whose full name matches one of ``patterns``,
    in first-seen order (dfloat/run/run.py:461-470): the classes a device
    placement must keep on one device."""
    names = []
    for full_name, module in model.named_modules():
        if any(re.fullmatch(p, full_name) for p in patterns):
            cls_name = type(module).__name__
            if cls_name not in names:
                names.append(cls_name)
    return names


def _write_model_size(dfloat_repo_id: str, rows) -> None:
    """model_size.csv as the reference's loaders write it
    (dfloat/run/run.py:522-535): the FP8 blocks' size before and after."""
    with open(os.path.join(dfloat_repo_id, "model_size.csv"), "w") as f:
        f.write("fp8_blocks,rest,total\n")
        for inc, exc, tot in rows:
            f.write(f"{inc},{exc},{tot}\n")


def _warn_if_on_cpu(model) -> None:
    if any(p.device.type == "cpu" for p in model.parameters()):
        print("Warning: Some model layers are on CPU. For inference, ensure the model is fully "
              "loaded onto CUDA-compatible GPUs.", file=stderr)


class DFloatModel:
    """Compressed causal LM from local directories (dfloat/run/run.py:483-566).

    ``dfloat_repo_id``: a local directory holding the compressor's output for
    a Hugging Face model (config.json with a ``dfloat_config`` entry,
    pattern_dict.json and the safetensors with the compressed buffers).
    ``model_name_or_path``: the original FP8 model, as a local directory.
    Nothing is downloaded: a missing ``dfloat_repo_id`` raises
    FileNotFoundError where the reference would call snapshot_download.
    Placement: ``device`` moves the whole model; otherwise ``device_map``
    "auto" spreads it over the visible GPUs with accelerate, keeping every
    compressed block on one device (get_no_split_classes).
    """

    @classmethod
    def from_pretrained(cls, dfloat_repo_id: str, dfloat_model_id: str, model_name_or_path: str,
                        device: Optional[str] = None, device_map: str = "auto",
                        max_memory: Optional[Dict[Union[int, str], Union[int, str]]] = None,
                        trust_remote_code: bool = True, **kwargs):
        from transformers import AutoConfig, AutoModelForCausalLM

        from dfloat.utils import report_model_size

        if not os.path.isdir(dfloat_repo_id):
            raise FileNotFoundError(f"{dfloat_repo_id} is not a local directory "
                                    f"(hub download of {dfloat_model_id} is not supported)")
        model = AutoModelForCausalLM.from_pretrained(
            model_name_or_path, trust_remote_code=trust_remote_code,
            dtype=kwargs.get("torch_dtype", torch.bfloat16),
            attn_implementation=kwargs.get("attn_implementation"), low_cpu_mem_usage=True)
        model.eval()
        config = AutoConfig.from_pretrained(dfloat_repo_id)
        if not hasattr(config, "dfloat_config"):
            raise ValueError(f"{dfloat_repo_id}/config.json has no dfloat_config entry")
        dfloat_config = dict(config.dfloat_config)
        with open(os.path.join(dfloat_repo_id, "pattern_dict.json")) as f:
            dfloat_config["pattern_dict"] = json.load(f)
        before = report_model_size(model, include_pattern=dfloat_config["pattern_dict"]["fp8"])
        load_and_replace_tensors_parallel(model, dfloat_repo_id, dfloat_config)
        total = report_model_size(model, include_pattern=None)[2]
        _write_model_size(dfloat_repo_id, [before, (total - before[1], before[1], total)])
        if device:
            model = model.to(device)
        else:
            if device_map != "auto":
                raise ValueError('device_map should be "auto" if no specific device is provided.')
            model = _dispatch_auto(model, max_memory)
        _warn_if_on_cpu(model)
        # transformers' FP8Linear modules (the quantized Linears of an HF FP8
        # checkpoint, fed by the decode hooks) run on the engine's FP8 linear
        bind_fp8_linears(model)
        return model


def _dispatch_auto(model, max_memory):
    """Spread ``model`` over the visible GPUs with accelerate, keeping each
    compressed block whole (dfloat/run/run.py:547-557)."""
    from accelerate import dispatch_model, infer_auto_device_map
    from accelerate.utils import get_balanced_memory

    from dfloat.const import get_default_no_split_pattern

    no_split = get_no_split_classes(model, get_default_no_split_pattern(type(model).__name__))
    max_memory = get_balanced_memory(model, max_memory=max_memory,
                                     no_split_module_classes=no_split)
    device_map = infer_auto_device_map(model, max_memory=max_memory,
                                       no_split_module_classes=no_split)
    return dispatch_model(model, device_map)


class DFloatDiffSynthModelFP8:
    """Compressed DiffSynth pipeline from a local directory
    (dfloat/run/run.py:569-729).

    The reference builds the pipeline itself from a hub name through
    DiffSynth (FLUX.1-dev, Wan2.1/2.2, Qwen-Image), which needs the network
    and the DiffSynth package.  Here ``model_name_or_path`` may instead be an
    already built pipeline (any ``nn.Module`` whose module names follow the
    pipeline's, e.g. ``ecf8_amd.dit.FluxPipeline``); a hub name is built
    through DiffSynth only if that package is importable.  Then, as the
    reference does: VRAM management is enabled when the pipeline offers it,
    dfloat_config.json and pattern_dict.json are read from
    ``dfloat_repo_id``, the per-block safetensors registered with their
    decode hooks, and the pipeline moved to ``device``.
    """

    @classmethod
    def from_pretrained(cls, dfloat_repo_id: str, dfloat_model_id: str, model_name_or_path,
                        device: Optional[str] = "cuda"):
        from dfloat.utils import report_model_size

        if not os.path.isdir(dfloat_repo_id):
            raise FileNotFoundError(f"{dfloat_repo_id} is not a local directory "
                                    f"(hub download of {dfloat_model_id} is not supported)")
        if isinstance(model_name_or_path, str):
            pipe = _diffsynth_pipeline(model_name_or_path)
        else:
            pipe = model_name_or_path
        if hasattr(pipe, "enable_vram_management"):
            pipe.device = device
            pipe.enable_vram_management(num_persistent_param_in_dit=0)
        with open(os.path.join(dfloat_repo_id, "dfloat_config.json")) as f:
            dfloat_config = json.load(f)
        with open(os.path.join(dfloat_repo_id, "pattern_dict.json")) as f:
            dfloat_config["pattern_dict"] = json.load(f)
        before = report_model_size(pipe, include_pattern=dfloat_config["pattern_dict"]["fp8"])
        load_and_replace_tensors_parallel(pipe, dfloat_repo_id, dfloat_config)
        total = report_model_size(pipe, include_pattern=None)[2]
        _write_model_size(dfloat_repo_id, [before, (total - before[1], before[1], total)])
        pipe.to(device)
        pipe.eval()
        _warn_if_on_cpu(pipe)
        return pipe


def _diffsynth_pipeline(model_name: str):
    try:
        import diffsynth  # noqa: F401
    except ImportError:
        raise ImportError(
            f"building the {model_name} pipeline needs the DiffSynth package, which is not "
            "installed; pass an already built pipeline as model_name_or_path") from None
    raise ValueError(f"{model_name}: pass the built DiffSynth pipeline as model_name_or_path "
                     "(pipelines are not downloaded)")
