"""The ctypes stub that the repository's integration guide gives a
maintainer of the reference (the block between its ``stub:begin`` /
``stub:end`` markers), run exactly as written: the reference's callers pass integer device addresses
(dfloat/run/run.py:104-119, scripts/compress.py:109-124).

CPU: against a stand-in library that records each call, the stub makes
the two calls of the C ABI with the caller's integers, torch's current
stream and the largest-block size taken from shared_mem.  GPU: against
libecf8.so, the stub's decode is bit-exact."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _stub_source() -> str:
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    block = re.search(r"<!-- stub:begin -->\s*```python\n(.*?)```\s*<!-- stub:end -->", text, re.S)
    assert block, "stub markers missing from INTEGRATION.md"
    return block.group(1)


class _Fn:
    def __init__(self, name, calls, ret=0):
        self.name, self.calls, self.ret = name, calls, ret
        self.argtypes, self.restype = None, None

    def __call__(self, *args):
        self.calls.append((self.name, args))
        return self.ret if self.name != "ecf8_status_string" else b"stand-in"


class _FakeLib:
    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        fn = _Fn(name, self.calls)
        setattr(self, name, fn)
        return fn


class _FakeStream:
    device = torch.device("cpu")
    cuda_stream = 0x5EED


def _exec_stub(monkeypatch, lib):
    monkeypatch.setattr(ctypes, "CDLL", lambda path: lib)
    ns = {}
    exec(compile(_stub_source(), "INTEGRATION.md:stub", "exec"), ns)
    return ns


def test_stub_passes_the_callers_integers_through(monkeypatch):
    fake = _FakeLib()
    ns = _exec_stub(monkeypatch, fake)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a: _FakeStream())
    args = [0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 3, 40_000, np.int64(123_456)]
    ns["_decode"](grid=(10,), block=(512,), shared_mem=512 * 4 + 4 + 12_345, args=args)
    (b_name, b_args), (d_name, d_args) = fake.calls
    assert b_name == "ecf8_build_table_cached" and d_name == "ecf8_decode"
    table = b_args[3]
    assert b_args == (0x1000, 3, -1, table, 0x5EED)
    assert d_args == (0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 3, 40_000, 123_456, 12_345,
                      0, table, -1, 512, 8, 0x5EED)
    assert all(type(a) is int for a in d_args if a is not None)
    # a second call with the same LUT address reuses the cache; other LUTs get their own
    ns["_decode"](grid=(10,), block=(512,), shared_mem=0, args=args)
    assert fake.calls[2][1][3] == table
    ns["_decode"](grid=(10,), block=(512,), shared_mem=0, args=[0x1100] + args[1:])
    assert fake.calls[4][1][3] != table
    assert len(ns["_tables"]) == 2


def test_stub_declarations_match_the_library_binding(monkeypatch):
    from ecf8_amd._lib import _SIGNATURES, ECF8_TABLE_ANY, ECF8_TABLE_CACHE_BYTES

    fake = _FakeLib()
    ns = _exec_stub(monkeypatch, fake)
    assert ns["ECF8_TABLE_CACHE_BYTES"] == ECF8_TABLE_CACHE_BYTES
    assert ns["ECF8_TABLE_ANY"] == ECF8_TABLE_ANY
    for name in ("ecf8_build_table_cached", "ecf8_decode"):
        assert getattr(fake, name).argtypes == _SIGNATURES[name][0], name


def test_stub_raises_on_a_failed_call(monkeypatch):
    fake = _FakeLib()
    ns = _exec_stub(monkeypatch, fake)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a: _FakeStream())
    fake.ecf8_decode.ret = 3
    with pytest.raises(RuntimeError, match="ecf8_decode: stand-in"):
        ns["_decode"](grid=(1,), block=(512,), shared_mem=0, args=[1, 2, 3, 4, 5, 6, 2, 7, 8])


@pytest.mark.gpu
def test_stub_decodes_bit_exact_on_the_gpu(monkeypatch, cuda_device):
    from dfloat.compress import compress_flat
    from ecf8_amd.build import LIB_PATH
    from ecf8_amd.synth import synthetic_fp8

    real = ctypes.CDLL
    monkeypatch.setattr(ctypes, "CDLL", lambda path: real(LIB_PATH if path == "libecf8.so" else path))
    ns = {}
    exec(compile(_stub_source(), "INTEGRATION.md:stub", "exec"), ns)
    w, _ = synthetic_fp8(384, 1024, 0.02, seed=9)
    flat = w.reshape(-1)
    res = compress_flat(flat)
    d = {k: res[k].contiguous().to(cuda_device) for k in
         ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")}
    op = res["output_positions"].numpy().view(np.uint64).astype(np.int64)
    out = torch.empty(flat.numel(), dtype=torch.float8_e4m3fn, device=cuda_device)
    n_bytes = d["encoded"].numel()
    call = dict(grid=(-(-n_bytes // 4096),), block=(512,),
                shared_mem=512 * 4 + 4 + int(np.diff(op).max()),
                args=[d["luts"].data_ptr(), d["encoded"].data_ptr(),
                      d["packed_other_4bits"].data_ptr(), d["output_positions"].data_ptr(),
                      d["gaps"].data_ptr(), out.data_ptr(), d["luts"].shape[0], n_bytes,
                      flat.numel()])
    for _ in range(2):  # the second call finds its table cached
        out.view(torch.uint8).zero_()
        ns["_decode"](**call)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.uint8).cpu(), flat.view(torch.uint8))
    assert len(ns["_tables"]) == 1


# --------------------------------------------- the tiled C-ABI block (ECF8-T)


def _tiled_source() -> str:
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    block = re.search(r"<!-- tiled:begin -->\s*```python\n(.*?)```\s*<!-- tiled:end -->", text,
                      re.S)
    assert block, "tiled markers missing from INTEGRATION.md"
    return block.group(1)


def test_tiled_block_declares_the_library_signatures(monkeypatch):
    from ecf8_amd._lib import _SIGNATURES

    fake = _FakeLib()
    monkeypatch.setattr(ctypes, "CDLL", lambda path: fake)
    ns = {}
    exec(compile(_tiled_source(), "INTEGRATION.md:tiled", "exec"), ns)
    for name in ("ecf8_code_from_luts", "ecf8_tile_sizes", "ecf8_tile_encode", "ecf8_build_table",
                 "ecf8_tile_linear"):
        assert getattr(fake, name).argtypes == _SIGNATURES[name][0], name
    assert [f for f, _ in ns["ecf8_tile_operand"]._fields_] == \
        ["stream", "seg_off", "gaps", "other", "weight_scale", "n", "out_col"]


@pytest.mark.gpu
def test_tiled_block_matches_the_fp8_linear_on_the_gpu(monkeypatch, cuda_device):
    """The block run as written: bit-identical to ecf8_fp8_linear over the
    Linear's FP8 weight; a block whose LUTs have a 1-bit code is refused
    before any tiled launch."""
    from dfloat.compress import compress_flat
    from ecf8_amd.build import LIB_PATH
    from ecf8_amd.llm_kernels import act_quant, fp8_linear
    from ecf8_amd.synth import flat_block, synthetic_block
    from ecf8_amd.tiled import linear_waves

    real = ctypes.CDLL
    monkeypatch.setattr(ctypes, "CDLL", lambda path: real(LIB_PATH if path == "libecf8.so" else path))
    ns = {}
    exec(compile(_tiled_source(), "INTEGRATION.md:tiled", "exec"), ns)
    weights = synthetic_block({"k_proj": (1024, 4096, 0.02), "o_proj": (512, 4096, 0.01)}, seed=4)
    res = compress_flat(flat_block(weights)[0])
    w, s = weights["k_proj"]
    dev = cuda_device
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(16, 4096, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    aq = torch.empty(16, 4096, dtype=torch.float8_e4m3fn, device=dev)
    a_s = torch.empty(16, 32, dtype=torch.float32, device=dev)
    act_quant(x, 16, aq, a_s)
    for M in (1, 7, 16):
        got = ns["tiled_linear"](res["luts"], w, s.to(dev), aq, a_s, M,
                                 linear_waves(1024, 4096, dev))
        want = torch.empty(M, 1024, dtype=torch.bfloat16, device=dev)
        fp8_linear(aq, a_s, [(w.to(dev), s.to(dev))], want, M)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), M
    # LUTs with a 1-bit code: refused, nothing launched
    b = w.view(torch.uint8).clone()
    b = (b & 0x87) | (11 << 3)
    b[::7] = (b[::7] & 0x87) | (12 << 3)
    skew = compress_flat(b.view(torch.float8_e4m3fn).reshape(-1))
    with pytest.raises(RuntimeError, match="no automaton"):
        ns["tiled_linear"](skew["luts"], b.view(torch.float8_e4m3fn), s.to(dev), aq, a_s, 1, 8)
