"""ctypes front end for oracle/liboracle.so (test infrastructure only).

Wraps the C restatement of the reference encoder (dfloat/utils.py:373-499)
and decode rule (dfloat/run/decode.cu:15-211).  ``build()`` compiles it with
the Makefile next to this file.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_encode.argtypes = [p, i64, p, p, i32, ctypes.c_uint32, i32, i32,
                                    p, i64, p, p, i64, p, p, i64, p, p, i64]
        L.oracle_encode.restype = i32
        L.oracle_decode_range.argtypes = [p, i32, p, i64, p, p, p, p, i64, i32, i32, i64, i64]
        L.oracle_decode_range.restype = i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def encode(exps: np.ndarray, table: dict, eof, bytes_per_thread=8, threads_per_block=512):
    """C restatement of the reference encoder; same outputs as
    oracle.codec.encode_exponents."""
    exps = np.ascontiguousarray(exps, dtype=np.uint8)
    n = exps.size
    code_bits = np.zeros(16, np.uint8)
    code_vals = np.zeros(16, np.uint32)
    for s, (bits, val) in table.items():
        if s is eof or not isinstance(s, (int, np.integer)):
            continue
        code_bits[int(s)] = bits
        code_vals[int(s)] = val
    eof_bits, eof_val = table[eof]
    total_bits = int(np.sum(code_bits[exps].astype(np.int64))) if n else 0
    enc_cap = total_bits // 8 + 2
    bytes_per_block = bytes_per_thread * threads_per_block
    blocks = -(-enc_cap // bytes_per_block)
    gap_cap = max(blocks * threads_per_block, 1)
    encoded = np.zeros(enc_cap, np.uint8)
    gaps = np.zeros(gap_cap // 2 + 1, np.uint8)
    op = np.zeros(blocks + 2, np.uint64)
    scratch = np.zeros(gap_cap, np.uint8)
    nb, ng, no = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    rc = lib().oracle_encode(_ptr(exps), n, _ptr(code_bits), _ptr(code_vals), eof_bits, eof_val,
                             bytes_per_thread, threads_per_block,
                             _ptr(encoded), enc_cap, ctypes.byref(nb),
                             _ptr(gaps), gaps.size, ctypes.byref(ng),
                             _ptr(op), op.size, ctypes.byref(no),
                             _ptr(scratch), scratch.size)
    if rc != 0:
        raise RuntimeError(f"oracle_encode failed: {rc}")
    return encoded[: nb.value].copy(), gaps[: ng.value].copy(), op[: no.value].copy()


def decode(luts, encoded, packed, output_positions, gaps, n_elements=None,
           threads_per_block=512, bytes_per_thread=8, threads=1, out=None):
    """C restatement of the decode rule; ``threads`` > 1 splits the
    format-blocks over a thread pool (ctypes releases the GIL)."""
    luts = np.ascontiguousarray(luts, dtype=np.uint8)
    encoded = np.ascontiguousarray(encoded, dtype=np.uint8)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    op = np.ascontiguousarray(np.asarray(output_positions).view(np.uint64))
    gaps = np.ascontiguousarray(gaps, dtype=np.uint8)
    n = packed.size * 2 if n_elements is None else int(n_elements)
    if out is None:
        out = np.zeros(n, np.uint8)
    blocks = -(-encoded.size // (threads_per_block * bytes_per_thread))
    n_luts = luts.shape[0] if luts.ndim == 2 else luts.size // 256
    L = lib()

    def run(rng):
        b0, b1 = rng
        rc = L.oracle_decode_range(_ptr(luts), n_luts, _ptr(encoded), encoded.size, _ptr(packed),
                                   _ptr(op), _ptr(gaps), _ptr(out), n, threads_per_block,
                                   bytes_per_thread, b0, b1)
        if rc != 0:
            raise RuntimeError(f"oracle_decode_range failed: {rc}")

    if threads <= 1 or blocks < 2:
        run((0, blocks))
    else:
        edges = np.linspace(0, blocks, threads + 1).astype(np.int64)
        with ThreadPoolExecutor(threads) as ex:
            list(ex.map(run, [(int(edges[i]), int(edges[i + 1])) for i in range(threads)]))
    return out
