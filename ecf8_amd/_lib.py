"""ctypes binding of libecf8.so (include/ecf8.h).

torch is imported first on purpose: the library links the HIP runtime by its
soname, so loading it after torch binds it to the runtime instance torch
already mapped, and torch's stream handles stay valid for its launches.
There is no fallback: a missing library raises ``ECF8Error``.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before libecf8.so)

from .build import LIB_PATH

ECF8_OK = 0
ECF8_TABLE_BYTES = 24624
ECF8_MAX_LUTS = 18
ECF8_TABLE_CACHE_BYTES = ECF8_TABLE_BYTES + 8 + ECF8_MAX_LUTS * 256
ECF8_TABLE_ANY = -1
ECF8_TABLE_MULTI = 0
ECF8_TABLE_DFA = 1


class ECF8Error(RuntimeError):
    """A libecf8 call failed, or the library is not built."""


_lib = None
_vp, _i64, _i32, _u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32
_f32 = ctypes.c_float

_SIGNATURES = {
    "ecf8_version": ([], ctypes.c_char_p),
    "ecf8_status_string": ([_i32], ctypes.c_char_p),
    "ecf8_decode_batched": ([_vp, _i32, _i32, _i32, _i64, _i32, _vp], _i32),
    "ecf8_decode_batched_select": ([_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i32, _vp], _i32),
    "ecf8_build_table_host": ([_vp, _i32, _i32, _vp, _vp], _i32),
    "ecf8_build_table": ([_vp, _i32, _i32, _vp, _vp, _vp], _i32),
    "ecf8_build_table_cached": ([_vp, _i32, _i32, _vp, _vp], _i32),
    "ecf8_decode": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _i32, _i32,
                     _i32, _vp], _i32),
    "ecf8_decode_noalloc": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp],
                            _i32),
    "ecf8_decode_bf16": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _i32, _vp, _i32,
                          _i32, _i32, _vp], _i32),
    "ecf8_encoded_sizes": ([_vp, _i64, _vp, _i32, _i32, _vp, _vp, _vp], _i32),
    "ecf8_encode_exponents": (
        [_vp, _i64, _vp, _vp, _i32, _u32, _i32, _i32, _vp, _i64, _vp, _i64, _vp, _i64],
        _i32,
    ),
    "ecf8_validate_format": (
        [_vp, _i32, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _i32, ctypes.c_char_p, ctypes.c_size_t],
        _i32,
    ),
    "ecf8_stream_probe": ([_i32, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp], _i32),
    # include/ecf8_tile.h: the tiled execution layout
    "ecf8_code_from_luts": ([_vp, _i32, _vp, _vp], _i32),
    "ecf8_tile_sizes": ([_vp, _i64, _i64, _vp, _vp, _vp], _i32),
    "ecf8_tile_encode": ([_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i32], _i32),
    "ecf8_tile_linear": ([_vp, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _i32, _vp], _i32),
    "ecf8_tile_decode": ([_vp, _i64, _vp, _vp, _vp], _i32),
    "ecf8_tile_moe_linear": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64,
                              _vp, _i64, _i32, _vp], _i32),
    "ecf8_tile_decode_batch": ([_vp, _vp, _vp, _i32, _i64, _i64, _vp], _i32),
    # include/ecf8_llm.h: the consumer kernels
    "ecf8_fp8_linear": ([_vp, _vp, _i64, _i64, _vp, _i32, _vp, _i64, _vp], _i32),
    "ecf8_rmsnorm": ([_vp, _vp, _vp, _f32, _i64, _i64, _vp, _vp, _vp, _vp], _i32),
    "ecf8_silu_mul_quant": ([_vp, _i64, _i64, _vp, _vp, _vp], _i32),
    "ecf8_act_quant": ([_vp, _i64, _i64, _vp, _vp, _vp], _i32),
    "ecf8_qk_norm_rope": ([_vp, _i64, _i64, _i32, _i32, _vp, _vp, _f32, _vp, _vp, _vp, _i64, _vp,
                           _vp, _vp, _vp], _i32),
    "ecf8_dequant_fp8_block": ([_vp, _vp, _i64, _i64, _vp, _vp], _i32),
    "ecf8_attention_work_floats": ([_i64, _i32, _i64], _i64),
    "ecf8_decode_attention": ([_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i64, _vp, _i64, _vp, _vp, _vp,
                               _vp], _i32),
    "ecf8_decode_attention_fused": ([_vp, _i64, _i32, _i32, _vp, _vp, _f32, _vp, _vp, _vp, _i64,
                                     _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp], _i32),
    "ecf8_moe_route": ([_vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "ecf8_moe_group": ([_vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "ecf8_moe_linear": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i32, _vp,
                         _i64, _vp], _i32),
    "ecf8_moe_combine": ([_vp, _i64, _vp, _vp, _i64, _i32, _i64, _vp, _vp], _i32),
}

EXPORTED = tuple(_SIGNATURES)


def lib():
    """Load libecf8.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ECF8Error(
                f"{LIB_PATH} is missing: build it with `python -m ecf8_amd.build` "
                "(there is no CPU fallback for the decode path)"
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def status_string(rc: int) -> str:
    return lib().ecf8_status_string(rc).decode()


def check(rc: int, what: str) -> None:
    if rc != ECF8_OK:
        raise ECF8Error(f"{what} failed: {status_string(rc)} (status {rc})")
