"""ECF8 codec API with the reference's names (dfloat/utils.py).

Offline, CPU-side producers of the decoder's input: FP8 split, block
flattening, codebook, decode LUTs and the bitstream encoder (the latter in
C++ inside libecf8, replacing the reference's per-symbol Python loop), plus
the module lookups and size report the compressor and loaders use.
"""

from __future__ import annotations

import ctypes
import re
from sys import stderr

import numpy as np
import torch

from .huffman import HuffmanCodec, get_nbit_codec  # noqa: F401  (re-exported API)

__all__ = [
    "flatten_block_of_weights",
    "get_exponents_and_other_4bits_fp8_e4m3",
    "compute_shannon_entropy",
    "get_nbit_codec",
    "get_luts_from_huffman_table",
    "encode_exponents_for_cuda",
    "locate_block_by_regex",
    "find_layers_by_data_type_and_layer_type",
    "find_layers_by_selection",
    "find_layers_by_layer_type",
    "find_layers_by_data_type",
    "param_to_bytes",
    "report_model_size",
    "repo_id_to_model_id",
]


# ------------------------------------------------------------------ layout


def flatten_block_of_weights(layers: dict, dtype=torch.float8_e4m3fn):
    """Concatenate the flattened ``.weight`` of each layer, in the dict's
    order (callers pass name-sorted dicts), and return (flat, split_positions)
    with split_positions = cumulative numels minus the last (int64).
    Follows dfloat/utils.py:188-204."""
    numels = [m.weight.numel() for m in layers.values()]
    flat = torch.empty(sum(numels), dtype=dtype)
    off = 0
    for m, k in zip(layers.values(), numels):
        flat[off : off + k] = m.weight.data.detach().reshape(-1)
        off += k
    split_positions = torch.cumsum(torch.tensor(numels, dtype=torch.int64), dim=0)[:-1]
    return flat, split_positions


def get_exponents_and_other_4bits_fp8_e4m3(data: torch.Tensor):
    """e4m3fn -> (4-bit exponents u8[n], packed sign|mantissa nibbles u8[n/2]).

    Exponent = bits 6..3 of each byte; the other nibble is sign (bit 7) over
    mantissa (bits 2..0); two nibbles per byte, even element high.
    Follows dfloat/utils.py:207-227."""
    assert data.ndim == 1
    assert data.dtype == torch.float8_e4m3fn
    w = data.view(torch.uint8)
    exps = (w >> 3) & 0xF
    other = ((w >> 4) & 0x8) | (w & 0x7)
    pairs = other.view(-1, 2)
    return exps, (pairs[:, 0] << 4) | pairs[:, 1]


def compute_shannon_entropy(data: torch.Tensor) -> float:
    """Shannon entropy in bits of the value histogram (dfloat/utils.py:230-236)."""
    assert data.ndim == 1
    _, freqs = torch.unique(data, return_counts=True)
    p = freqs / freqs.sum()
    return float(-torch.sum(p * torch.log2(p)).item())


# -------------------------------------------------------------------- LUTs


def get_luts_from_huffman_table(table: dict) -> torch.Tensor:
    """Two-level decode tables u8[n_luts, 256] (dfloat/utils.py:270-370).

    Row 0 maps a code's first byte: codes of <= 8 bits to their symbol,
    longer codes to the pointer value 256 - r of the row r that holds their
    first byte (rows in first-appearance order over the table).  Row r maps
    the second byte of the codes starting with that first byte.  Every key is
    the code left-justified to the byte, and each row is filled forward from
    its keys (entries before the first key hold 0).  The last row is the code
    length per symbol.
    """
    codes = [(int(s), b, v) for s, (b, v) in table.items() if isinstance(s, (int, np.integer))]
    if any(b > 16 for _, b, _ in codes):
        raise ValueError("codes longer than 16 bits cannot be represented by two LUT levels")
    first_bytes = []
    for _, bits, val in codes:
        if bits > 8:
            fb = val >> (bits - 8)
            if fb not in first_bytes:
                first_bytes.append(fb)
    n_rows = 1 + len(first_bytes)
    keyed = [dict() for _ in range(n_rows)]

    def put(row, key, value):
        old = keyed[row].get(key)
        if old is not None and old != value:
            raise ValueError(f"Key {key} already exists in {keyed[row]}")
        keyed[row][key] = value

    for sym, bits, val in codes:
        if bits <= 8:
            put(0, val << (8 - bits), sym)
        else:
            fb = val >> (bits - 8)
            r = 1 + first_bytes.index(fb)
            put(0, fb, 256 - r)
            put(r, (val << (16 - bits)) & 0xFF, sym)

    luts = np.zeros((n_rows + 1, 256), dtype=np.uint8)
    for r in range(n_rows):
        if not keyed[r]:
            continue
        keys = np.array(sorted(keyed[r]), dtype=np.int64)
        vals = np.array([keyed[r][k] for k in keys], dtype=np.uint8)
        # forward fill: entry k holds the value of the last key <= k
        idx = np.searchsorted(keys, np.arange(256), side="right") - 1
        luts[r] = np.where(idx >= 0, vals[np.maximum(idx, 0)], 0)
    for sym, bits, _ in codes:
        luts[n_rows, sym] = bits
    return torch.from_numpy(luts)


# ------------------------------------------------------------------ encoder


def _code_arrays(codec):
    table = codec._table
    bits = np.zeros(16, np.uint8)
    vals = np.zeros(16, np.uint32)
    for s, (b, v) in table.items():
        if isinstance(s, (int, np.integer)):
            if not 0 <= int(s) <= 15:
                raise ValueError(f"symbol {s} is not a 4-bit exponent")
            bits[int(s)] = b
            vals[int(s)] = v
    eof_bits, eof_val = table[codec._eof]
    return bits, vals, int(eof_bits), int(eof_val)


def encode_exponents_for_cuda(exponents_4bits, codec, bytes_per_thread: int = 8,
                              threads_per_block: int = 512):
    """Encode 4-bit exponents into (encoded u8, gaps u8, output_positions u64)
    torch tensors; same outputs as dfloat/utils.py:502-530, computed by the
    C++ encoder in libecf8 (ecf8_encode_exponents)."""
    from ecf8_amd._lib import check, lib

    if isinstance(exponents_4bits, torch.Tensor):
        exps = exponents_4bits.detach().to("cpu", torch.uint8).contiguous().numpy()
    else:
        exps = np.ascontiguousarray(exponents_4bits, dtype=np.uint8)
    bits, vals, eof_bits, eof_val = _code_arrays(codec)
    L = lib()
    n = exps.size
    nb, ng, no = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    check(L.ecf8_encoded_sizes(vp(exps), n, vp(bits), bytes_per_thread, threads_per_block,
                               ctypes.byref(nb), ctypes.byref(ng), ctypes.byref(no)),
          "ecf8_encoded_sizes")
    encoded = np.zeros(max(nb.value, 1), np.uint8)
    gaps = np.zeros(max(ng.value, 1), np.uint8)
    op = np.zeros(no.value, np.uint64)
    check(L.ecf8_encode_exponents(vp(exps), n, vp(bits), vp(vals), eof_bits, eof_val,
                                  bytes_per_thread, threads_per_block, vp(encoded), nb.value,
                                  vp(gaps), ng.value, vp(op), no.value),
          "ecf8_encode_exponents")
    return (torch.from_numpy(encoded[: nb.value].copy()),
            torch.from_numpy(gaps[: ng.value].copy()),
            torch.from_numpy(op))


# ------------------------------------------------------------ block lookup


def locate_block_by_regex(model, pattern):
    """Modules whose full name matches ``pattern`` (dfloat/utils.py:75-80)."""
    return {name: m for name, m in model.named_modules() if re.fullmatch(pattern, name)}


def find_layers_by_data_type_and_layer_type(module, target_dtype=torch.bfloat16,
                                            layers=(torch.nn.Linear, torch.nn.Embedding),
                                            name=""):
    """Name-sorted {name: module} of the first modules of the given types whose
    weight has ``target_dtype`` (dfloat/utils.py:158-185)."""
    if (type(module) in tuple(layers) and hasattr(module, "weight")
            and getattr(module.weight, "dtype", None) == target_dtype):
        return {name: module}
    res = {}
    for child_name, child in module.named_children():
        full = f"{name}.{child_name}" if name else child_name
        res.update(find_layers_by_data_type_and_layer_type(child, target_dtype, layers, full))
    return dict(sorted(res.items()))


def find_layers_by_selection(module, select, name=""):
    """Name-sorted {name: module} of the attribute paths in ``select`` found
    under ``module`` or any descendant (dfloat/utils.py:83-117)."""
    res = {}
    for path in select:
        target = module
        try:
            for part in path.split("."):
                target = getattr(target, part)
        except AttributeError:
            continue
        res[f"{name}.{path}" if name else path] = target
    for child_name, child in module.named_children():
        full = f"{name}.{child_name}" if name else child_name
        res.update(find_layers_by_selection(child, select, full))
    return dict(sorted(res.items()))


def find_layers_by_layer_type(module, layers=(torch.nn.Linear,), name=""):
    """Name-sorted {name: module} of the outermost modules whose type is one
    of ``layers`` (dfloat/utils.py:120-132)."""
    if type(module) in tuple(layers):
        return {name: module}
    res = {}
    for child_name, child in module.named_children():
        full = f"{name}.{child_name}" if name else child_name
        res.update(find_layers_by_layer_type(child, layers, full))
    return dict(sorted(res.items()))


def find_layers_by_data_type(module, target_dtype=torch.bfloat16, name=""):
    """Name-sorted {name: module} of the outermost modules whose ``weight``
    has ``target_dtype`` (dfloat/utils.py:135-155)."""
    if getattr(getattr(module, "weight", None), "dtype", None) == target_dtype:
        return {name: module}
    res = {}
    for child_name, child in module.named_children():
        full = f"{name}.{child_name}" if name else child_name
        res.update(find_layers_by_data_type(child, target_dtype, full))
    return dict(sorted(res.items()))


# ------------------------------------------------------------- size report

_ELEMENT_BYTES = {
    1: (torch.uint8, torch.int8, torch.float8_e4m3fn),
    2: (torch.float16, torch.bfloat16, torch.int16, torch.uint16),
    4: (torch.float32, torch.int32, torch.uint32),
    8: (torch.float64, torch.int64, torch.uint64),
}


def param_to_bytes(param) -> int:
    """Storage bytes of a tensor for the dtypes a checkpoint holds
    (dfloat/utils.py:11-21); ValueError for any other dtype."""
    for size, dtypes in _ELEMENT_BYTES.items():
        if param.dtype in dtypes:
            return param.numel() * size
    raise ValueError(f"Unrecognized parameter data type {param.dtype}.")


def _included(name: str, include_pattern) -> bool:
    if isinstance(include_pattern, list):
        return any(re.search(p, name) for p in include_pattern)
    for pattern, attrs in include_pattern.items():
        if re.search(pattern, name) and any(a in name for a in (attrs or ())):
            return True
    return False


def report_model_size(model, include_pattern):
    """(included GiB, excluded GiB, total GiB) of ``model.state_dict()``
    (dfloat/utils.py:24-67).  ``include_pattern``: a list of regexes searched
    in each state-dict name; a dict {regex: attribute names}, where a name
    counts when it matches the regex and contains one of the attributes; or
    None (everything included).  The three figures go to stderr."""
    if include_pattern is not None and not isinstance(include_pattern, (list, dict)):
        raise ValueError("`include_pattern` must be either a list of strings or a dictionary, "
                         "or None")
    inc = exc = 0
    for name, tensor in model.state_dict().items():
        if include_pattern is None or _included(name, include_pattern):
            inc += param_to_bytes(tensor)
        else:
            exc += param_to_bytes(tensor)
    gib = 1024 ** 3
    inc_gb, exc_gb, tot_gb = inc / gib, exc / gib, (inc + exc) / gib
    print(f"Included model size: {inc_gb:0.4f} GB", file=stderr)
    print(f"Excluded model size: {exc_gb:0.4f} GB", file=stderr)
    print(f"Total model size: {tot_gb:0.4f} GB", file=stderr)
    return inc_gb, exc_gb, tot_gb


def repo_id_to_model_id(repo_id: str) -> str:
    """Hub cache directory name of a repo id: "org/name" -> "models--org--name"
    (dfloat/utils.py:70-72)."""
    return "models--" + "--".join(repo_id.split("/"))
