"""The C-ABI library loads, binds torch's HIP runtime, exports every function
the headers under include/ declare, and rejects bad arguments before
touching the GPU.  CPU only: no call here reaches a HIP API."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
HEADER = os.path.join(INCLUDE, "ecf8.h")


def _declared_functions():
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if h.endswith(".h"):
            text = re.sub(r"/\*.*?\*/", "", open(os.path.join(INCLUDE, h)).read(), flags=re.S)
            names |= set(re.findall(r"\b(ecf8_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_binding_table():
    from ecf8_amd._lib import EXPORTED

    assert _declared_functions() == sorted(EXPORTED)


def test_library_exports_every_declared_symbol():
    from ecf8_amd._lib import lib

    L = lib()
    for name in _declared_functions():
        assert hasattr(L, name), name
    assert L.ecf8_version().decode().startswith("ecf8_amd")


def test_single_hip_runtime_mapped():
    import torch  # noqa: F401

    from ecf8_amd._lib import lib

    lib()
    maps = open("/proc/self/maps").read()
    runtimes = set(re.findall(r"(/\S*libamdhip64\S*)", maps))
    assert len(runtimes) == 1, runtimes


def test_status_strings():
    from ecf8_amd._lib import lib

    L = lib()
    assert L.ecf8_status_string(0) == b"ok"
    assert L.ecf8_status_string(3) == b"misaligned device buffer"


def _decode_call(**kw):
    from ecf8_amd._lib import lib

    args = dict(luts=0x1000, encoded=0x2000, packed=0x3000, op=0x4000, gaps=0x5000, out=0x6000,
                n_luts=3, n_bytes=100, n=64, table=0x7000, kind=1, tpb=512, bpt=8)
    args.update(kw)
    return lib().ecf8_decode(args["luts"], args["encoded"], args["packed"], args["op"],
                             args["gaps"], args["out"], args["n_luts"], args["n_bytes"], args["n"],
                             0, 0, args["table"], args["kind"], args["tpb"], args["bpt"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(bpt=4), 2),           # geometry the reference kernel does not have
    (dict(tpb=300), 2),
    (dict(n=63), 1),            # odd element count
    (dict(n_bytes=-1), 1),
    (dict(n_luts=1), 4),
    (dict(n_luts=19), 4),
    (dict(out=0x6001), 3),      # 16-byte output alignment
    (dict(encoded=0x2008), 3),  # 16-byte bitstream alignment
    (dict(n_bytes=2**31), 2),   # positions are 32-bit, as in the reference
    (dict(n=2**31), 2),
    (dict(n=2**31 - 64), 2),    # the last 64 below 2^31 are kept clear of the clamped loads
    (dict(packed=0x3002), 3),
    (dict(gaps=0), 1),
    (dict(kind=2), 1),          # unknown table kind
    (dict(kind=-2), 1),
])
def test_decode_rejects_before_launch(kw, status):
    assert _decode_call(**kw) == status


def test_decode_of_empty_block_is_a_no_op():
    assert _decode_call(n_bytes=0, n=0) == 0


def test_build_table_rejects_bad_lut_count():
    from ecf8_amd._lib import lib

    kind = ctypes.c_int()
    assert lib().ecf8_build_table(ctypes.c_void_p(0x1000), 19, -1, ctypes.c_void_p(0x2000),
                                  ctypes.byref(kind), None) == 4
    assert lib().ecf8_build_table(None, 3, -1, ctypes.c_void_p(0x2000), ctypes.byref(kind),
                                  None) == 1
    assert lib().ecf8_build_table(ctypes.c_void_p(0x1001), 3, -1, ctypes.c_void_p(0x2000),
                                  ctypes.byref(kind), None) == 3
    assert lib().ecf8_build_table(ctypes.c_void_p(0x1000), 3, 7, ctypes.c_void_p(0x2000),
                                  ctypes.byref(kind), None) == 1
    # an automaton-only table must be able to report a refusal to the host
    assert lib().ecf8_build_table(ctypes.c_void_p(0x1000), 3, 1, ctypes.c_void_p(0x2000),
                                  None, None) == 1


@pytest.mark.parametrize("args,status", [
    ((0x1000, -1, 1, 16, 0, 512), 1),      # negative count
    ((0x1000, 1, 1, 0, 0, 512), 1),        # blocks_per_task < 1
    ((0x1000, 1, 1, 16, 0, 300), 2),       # block size the kernels do not run
    ((0x1004, 1, 1, 16, 0, 512), 3),       # descriptors not 8-byte aligned
    ((None, 1, 1, 16, 0, 512), 1),
    ((None, 0, 0, 16, 0, 512), 0),         # nothing to do
])
def test_batched_decode_rejects_before_launch(args, status):
    from ecf8_amd._lib import lib

    assert lib().ecf8_decode_batched(*args, None) == status


def test_block_descriptor_layout_matches_the_header():
    import numpy as np

    from ecf8_amd.decode import BLOCK_DESC_DTYPE

    text = open(HEADER).read()
    struct = text[text.index("typedef struct ecf8_block_desc"):text.index("} ecf8_block_desc;")]
    fields = re.findall(r"\b(\w+);", struct)
    assert fields == list(BLOCK_DESC_DTYPE.names)
    assert BLOCK_DESC_DTYPE.itemsize == 80 and "80 bytes" in text
    assert [BLOCK_DESC_DTYPE.fields[f][1] for f in fields] == [0, 8, 16, 24, 32, 40, 48, 56, 64,
                                                               72, 76]
    assert np.dtype("<i4").itemsize == 4


def test_consumer_kernels_reject_before_launch():
    """include/ecf8_llm.h entry points check arguments before any HIP call."""
    import ctypes

    from ecf8_amd._lib import lib
    from ecf8_amd.llm_kernels import _Seg

    L = lib()
    fake = 1 << 20  # never dereferenced: every call below is rejected first
    seg = (_Seg * 1)(_Seg(fake, fake, 128, 0))
    assert L.ecf8_fp8_linear(None, fake, 16, 4096, seg, 1, fake, 128, None) == 1
    assert L.ecf8_fp8_linear(fake, fake, 16, 4000, seg, 1, fake, 128, None) == 2   # K % 128
    assert L.ecf8_fp8_linear(fake, fake, 16, 4096, seg, 4, fake, 128, None) == 1   # > 3 segments
    assert L.ecf8_fp8_linear(fake + 1, fake, 16, 4096, seg, 1, fake, 128, None) == 3
    assert L.ecf8_fp8_linear(fake, fake, 16, 4096, seg, 1, fake, 64, None) == 6    # ldo too small
    bad_n = (_Seg * 1)(_Seg(fake, fake, 100, 0))
    assert L.ecf8_fp8_linear(fake, fake, 16, 4096, bad_n, 1, fake, 128, None) == 2
    bad_layout = (_Seg * 1)(_Seg(fake, fake, 128, 0, 2))
    assert L.ecf8_fp8_linear(fake, fake, 16, 4096, bad_layout, 1, fake, 128, None) == 1
    assert L.ecf8_rmsnorm(None, None, fake, ctypes.c_float(1e-6), 4, 4096, fake, fake, None, None) == 1
    assert L.ecf8_rmsnorm(None, fake, fake, ctypes.c_float(1e-6), 4, 4096, None, fake, None, None) == 1
    assert L.ecf8_rmsnorm(None, fake, fake, ctypes.c_float(1e-6), 4, 4096, fake, None, fake, None) == 1
    assert L.ecf8_rmsnorm(None, fake, fake, ctypes.c_float(1e-6), 4, 3072, fake, fake, None, None) == 2
    assert L.ecf8_silu_mul_quant(fake, 4, 1000, fake, fake, None) == 2
    assert L.ecf8_act_quant(fake, 4, 4096, None, fake, None) == 1
    assert L.ecf8_qk_norm_rope(fake, 1, 1, 32, 8, fake, fake, ctypes.c_float(1e-6), fake, fake,
                               None, 64, fake, fake, fake, None) == 1
    assert L.ecf8_attention_work_floats(2, 32, 300) == 2 * 32 * 2 * 130
    assert L.ecf8_attention_work_floats(0, 32, 300) == -1
    assert L.ecf8_decode_attention(fake, fake, fake, fake, 2, 32, 16, 300, fake, 10 ** 6, fake,
                                   fake, None, None) == 2   # Hq != 4 Hkv
    assert L.ecf8_decode_attention(fake, fake, fake, fake, 2, 32, 8, 300, fake, 10, fake, fake,
                                   None, None) == 6         # work too small
    fa = L.ecf8_decode_attention_fused
    eps = ctypes.c_float(1e-6)
    assert fa(None, 2, 32, 8, fake, fake, eps, fake, fake, fake, 300, fake, fake, fake, 10 ** 6,
              fake, fake, None, None) == 1
    assert fa(fake, 2, 32, 16, fake, fake, eps, fake, fake, fake, 300, fake, fake, fake, 10 ** 6,
              fake, fake, None, None) == 2          # Hq / Hkv = 2
    assert fa(fake, 2, 32, 8, fake, fake, eps, fake, fake, fake, 300, fake, fake, fake,
              2 * 32 * 2 * 130 - 1, fake, fake, None, None) == 6   # work too small
    assert fa(fake, 2, 32, 8, fake, fake, eps, fake, fake, fake, 300, fake, fake, fake + 4,
              10 ** 6, fake, fake, None, None) == 3                # work 8-byte aligned


def test_batched_select_rejects_before_launch():
    from ecf8_amd._lib import lib

    L = lib()
    fake = 1 << 20
    f = L.ecf8_decode_batched_select
    assert f(fake, -1, fake, fake, fake, 4, 0, 512, None) == 1
    assert f(fake, 3, fake, fake, fake, 0, 0, 512, None) == 1       # blocks_per_task < 1
    assert f(fake, 0, None, None, None, 4, 0, 512, None) == 0       # nothing to do
    assert f(fake, 3, None, fake, fake, 4, 0, 512, None) == 1
    assert f(fake + 4, 3, fake, fake, fake, 4, 0, 512, None) == 3  # descs misaligned
    assert f(fake, 3, fake + 2, fake, fake, 4, 0, 512, None) == 3  # flags misaligned
    assert f(fake, 3, fake, fake, fake, 4, 0, 300, None) == 2


def test_moe_kernels_reject_before_launch():
    from ecf8_amd._lib import lib

    L = lib()
    fake = 1 << 20
    rt = L.ecf8_moe_route
    assert rt(None, fake, 16, 2048, 128, 8, fake, fake, fake, None) == 1
    assert rt(fake, fake, 16, 2048, 128, 8, None, fake, fake, None) == 1     # no logits buffer
    assert rt(fake, fake, 16, 1000, 128, 8, fake, fake, fake, None) == 2     # H % 512
    assert rt(fake, fake, 16, 2048, 300, 8, fake, fake, fake, None) == 2     # E > 256
    assert rt(fake, fake, 16, 2048, 128, 20, fake, fake, fake, None) == 2    # top_k > 16
    assert rt(fake, fake, 1 << 17, 2048, 128, 8, fake, fake, fake, None) == 2
    assert rt(fake + 2, fake, 16, 2048, 128, 8, fake, fake, fake, None) == 3
    g = L.ecf8_moe_group
    assert g(None, fake, 16, 8, 128, fake, fake, fake, fake, fake, fake, None, None) == 1
    assert g(fake, fake, 1100, 8, 128, fake, fake, fake, fake, fake, fake, None, None) == 2  # P > 8192
    lin = L.ecf8_moe_linear
    assert lin(None, fake, None, fake, fake, fake, 128, fake, fake, 2, 768, 2048, 0, fake, 1536,
               None) == 1
    assert lin(fake, fake, None, fake, fake, fake, 128, fake, fake, 2, 700, 2048, 0, fake, 1536,
               None) == 2   # seg_n % 128
    assert lin(fake, fake, None, fake, fake, fake, 128, fake, fake, 2, 768, 2048, 0, fake, 1000,
               None) == 6   # ldo < n_segs * seg_n
    assert lin(fake + 4, fake, None, fake, fake, fake, 128, fake, fake, 2, 768, 2048, 0, fake,
               1536, None) == 3
    assert lin(fake, fake, None, fake, fake, fake, 128, fake, fake, 2, 768, 2048, 2, fake, 1536,
               None) == 1   # unknown weight layout
    c = L.ecf8_moe_combine
    assert c(fake, 1024, fake, fake, 16, 8, 2048, fake, None) == 1   # ldd < H
    assert c(fake, 2052, fake, fake, 16, 8, 2052, fake, None) == 2   # H % 8
    assert c(fake + 2, 2048, fake, fake, 16, 8, 2048, fake, None) == 3
