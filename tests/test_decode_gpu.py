"""GPU parity of the HIP decoder: bit-exact against the original FP8 bytes
(the reference's own check, scripts/compress.py:126), the CPU oracle's
decode (oracle/, restating dfloat/run/decode.cu) and the golden vectors."""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import codec as oc

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
CASES = sorted(json.load(open(os.path.join(GOLDEN, "index.json"))))
KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev_block(block, dev):
    out = {}
    for k in KEYS:
        v = block[k]
        t = torch.from_numpy(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v
        out[k] = t.contiguous().to(dev)
    return out


ANY, MULTI, DFA = -1, 0, 1


def _table_for(d, kind):
    """Device table of the requested kind.  The automaton holds at most 4
    symbols per input byte, so LUTs with a 1-bit code refuse it: then the
    refusal is checked and the automatic choice (the multi-symbol table) is
    returned instead."""
    from ecf8_amd.decode import ECF8Error, build_table, min_code_bits

    try:
        return build_table(d["luts"], kind=kind)
    except ECF8Error:
        if kind != DFA:
            raise
    assert min_code_bits(d["luts"]) == 1, "automaton refused LUTs without a 1-bit code"
    table = build_table(d["luts"], kind=ANY)
    assert table.kind == MULTI
    return table


def _gpu_decode(block, dev, tpb=512, n_elements=None, out=None, kind=ANY):
    from ecf8_amd.decode import decode, decode_into

    d = _dev_block(block, dev)
    table = _table_for(d, kind)
    if out is None and n_elements is None:
        r = decode(d["luts"], d["encoded"], d["packed_other_4bits"], d["output_positions"],
                   d["gaps"], table=table, threads_per_block=tpb)
    else:
        r = decode_into(out, d["luts"], d["encoded"], d["packed_other_4bits"],
                        d["output_positions"], d["gaps"], table=table, threads_per_block=tpb,
                        n_elements=n_elements)
    torch.cuda.synchronize()
    return r.view(torch.uint8).cpu().numpy()


def _compress(flat_u8: np.ndarray, tpb=512):
    from dfloat.compress import compress_flat

    flat = torch.from_numpy(np.ascontiguousarray(flat_u8)).view(torch.float8_e4m3fn)
    res = compress_flat(flat, 8, tpb)
    return {k: res[k] for k in KEYS}


# ----------------------------------------------------------------- golden


@pytest.mark.parametrize("kind", [MULTI, DFA])
@pytest.mark.parametrize("name", CASES)
def test_golden_blocks_decode_bit_exact(name, kind, cuda_device):
    _say(f"golden {name} kind={kind}")
    g = dict(np.load(os.path.join(GOLDEN, f"{name}.npz")))
    got = _gpu_decode(g, cuda_device, tpb=int(g["threads_per_block"]), kind=kind)
    assert np.array_equal(got, g["flat"])


# ------------------------------------------------------------ distributions


def _random_block(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 60000)) * 2
    kind = seed % 5
    if kind == 0:
        k = int(rng.integers(1, 17))
        syms = rng.choice(16, k, replace=False)
        p = rng.pareto(0.5 + rng.random() * 2, k) + 1e-3
        exps = rng.choice(syms, n, p=p / p.sum()).astype(np.uint8)
    elif kind == 1:  # geometric: long codes, 1-bit codes
        exps = np.minimum(rng.geometric(0.5 + 0.45 * rng.random(), n) - 1, 15).astype(np.uint8)
    elif kind == 2:
        exps = np.full(n, int(rng.integers(0, 16)), np.uint8)
    elif kind == 3:
        exps = rng.integers(0, 16, n, dtype=np.uint8)
    else:
        w = rng.normal(0, 0.02, n).astype(np.float32)
        w = w / (np.abs(w).max() / 448.0)
        return torch.from_numpy(w).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()
    other = rng.integers(0, 16, n, dtype=np.uint8)
    return (((other & 8) << 4) | (exps << 3) | (other & 7)).astype(np.uint8)


@pytest.mark.parametrize("kind", [MULTI, DFA])
@pytest.mark.parametrize("seed", range(40))
def test_random_blocks_bit_exact_vs_original_and_oracle(seed, kind, cuda_device, oracle_native):
    flat = _random_block(seed)
    tpb = (128, 256, 512, 1024)[seed % 4]
    _say(f"random seed={seed} n={flat.size} tpb={tpb} kind={kind}")
    block = _compress(flat, tpb)
    got = _gpu_decode(block, cuda_device, tpb=tpb, kind=kind)
    want = oracle_native.decode(block["luts"].numpy(), block["encoded"].numpy(),
                                block["packed_other_4bits"].numpy(),
                                block["output_positions"].numpy(), block["gaps"].numpy(),
                                threads_per_block=tpb)
    assert np.array_equal(want, flat)
    assert np.array_equal(got, flat)


@pytest.mark.parametrize("kind", [MULTI, DFA])
def test_config1_4096x4096_bit_exact(kind, cuda_device, oracle_native):
    from ecf8_amd.synth import synthetic_fp8

    _say(f"config1 4096x4096 kind={kind}")
    w, _ = synthetic_fp8(4096, 4096, 0.02, seed=0)
    flat = w.reshape(-1).view(torch.uint8).numpy()
    block = _compress(flat)
    got = _gpu_decode(block, cuda_device, kind=kind)
    assert np.array_equal(got, flat)
    want = oracle_native.decode(*(block[k].numpy() for k in KEYS), threads=8)
    assert np.array_equal(want, got)


@pytest.fixture(scope="module")
def qwen3_layer_flat():
    """One Qwen3-8B-shaped layer's weights, flattened in the reference's
    order (uint8 view)."""
    from ecf8_amd.synth import flat_block, qwen3_8b_layer

    flat, _ = flat_block(qwen3_8b_layer(seed=0))
    return flat.view(torch.uint8)


def test_config2_qwen3_layer_bit_exact(cuda_device, qwen3_layer_flat):
    from ecf8_amd.decode import build_table

    _say("config2 qwen3-8b layer")
    flat_u8 = qwen3_layer_flat.numpy()
    block = _compress(flat_u8)
    d = _dev_block(block, cuda_device)
    assert build_table(d["luts"]).kind == DFA  # the automaton runs this workload
    for kind in (DFA, MULTI):
        _say(f"config2 kind={kind}")
        got = _gpu_decode(block, cuda_device, kind=kind)
        assert got.size == 192_937_984
        assert np.array_equal(got, flat_u8)


def test_largest_block_the_format_allows(cuda_device, qwen3_layer_flat):
    """One block of 2^31 - 2^17 elements, near the format's limit (32-bit
    element and byte counts, dfloat/run/decode.cu:23-25; the host refuses
    more than 2^31 - 65): the Qwen3 layer tiled 12 times, compressed as one
    block, decoded bit-exact by the automaton kernel.  Positions past 2^30
    exercise the kernel's 32-bit position arithmetic."""
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table, decode_into, largest_block, min_code_bits

    n = 2 ** 31 - 2 ** 17
    reps = -(-n // qwen3_layer_flat.numel())
    big = qwen3_layer_flat.repeat(reps)[:n]
    _say(f"largest block: compressing {n} elements")
    res = compress_flat(big.view(torch.float8_e4m3fn))
    d = {k: res[k].contiguous().to(cuda_device) for k in KEYS}
    table = build_table(d["luts"])
    assert table.kind == DFA
    out = torch.empty(n + 4096, dtype=torch.uint8, device=cuda_device)
    out[n:] = 0x5A
    _say("largest block: decoding")
    decode_into(out, d["luts"], d["encoded"], d["packed_other_4bits"], d["output_positions"],
                d["gaps"], table=table, n_elements=n,
                max_block_elements=largest_block(d["output_positions"]),
                min_code_bits=min_code_bits(d["luts"]))
    torch.cuda.synchronize()
    assert torch.equal(out[:n], big.to(cuda_device))
    assert bool((out[n:] == 0x5A).all())


@pytest.mark.parametrize("kind", [MULTI, DFA])
def test_corrupt_table_stays_inside_the_output(kind, cuda_device):
    """A table of random bits (a corrupt buffer, or one of the other kind)
    decodes garbage, but the kernels force its fields into range: nothing is
    written outside [0, n) and the launch completes."""
    from ecf8_amd.decode import DecodeTable, decode_into

    flat = _random_block(24)
    block = _compress(flat)
    d = _dev_block(block, cuda_device)
    rng = np.random.default_rng(5 + kind)
    junk = rng.integers(0, 2**32, 24608 // 4, dtype=np.uint64).astype(np.uint32)
    n = flat.size
    for table in (junk, _table_for(d, 1 - kind).data.cpu().numpy().view(np.uint32)):
        t = DecodeTable(torch.from_numpy(table.view(np.int32)).to(cuda_device), kind)
        out = torch.full((n + 512,), 0x77, dtype=torch.uint8, device=cuda_device)
        decode_into(out[:n], d["luts"], d["encoded"], d["packed_other_4bits"],
                    d["output_positions"], d["gaps"], table=t)
        torch.cuda.synchronize()
        assert (out[n:].cpu().numpy() == 0x77).all()


def _config_blocks():
    from ecf8_amd import synth

    return [
        ("qwen3-8b-layer-seed7", synth.QWEN3_8B_LAYER, 7),        # full-model layers
        ("flux-double-block", synth.FLUX_DOUBLE_BLOCK, 1),        # DiT
        ("flux-single-block", synth.FLUX_SINGLE_BLOCK, 2),
        ("qwen3-moe-attention", synth.QWEN3_MOE_ATTN, 3),         # MoE
        ("qwen3-moe-expert", synth.QWEN3_MOE_EXPERT, 4),
    ]


@pytest.mark.parametrize("name,shapes,seed", _config_blocks(), ids=[c[0] for c in _config_blocks()])
def test_config_blocks_bit_exact(name, shapes, seed, cuda_device):
    """One compressed block of each model family's shapes (the blocks the
    reference's pattern dicts cut: a decoder layer, a DiT double/single
    block, an MoE attention block and one expert) decodes bit-exactly."""
    from ecf8_amd.decode import build_table
    from ecf8_amd.synth import flat_block, synthetic_block

    _say(f"config block {name}")
    flat, _ = flat_block(synthetic_block(shapes, seed))
    flat_u8 = flat.view(torch.uint8).numpy()
    block = _compress(flat_u8)
    assert build_table(_dev_block(block, cuda_device)["luts"]).kind == DFA
    got = _gpu_decode(block, cuda_device)
    assert np.array_equal(got, flat_u8)


def test_dfa_exact_path_is_bit_exact(cuda_device):
    """Chunks whose automaton walk reaches the exact row are decoded with the
    LUT rule itself.  Valid streams only get there in their final padding,
    so here a copy of the automaton sends every chunk whose first byte is
    odd there; the output must not change."""
    from ecf8_amd.decode import DecodeTable, build_table_host, decode

    flat = _random_block(24)
    block = _compress(flat)
    d = _dev_block(block, cuda_device)
    table, kind = build_table_host(block["luts"], DFA)
    assert kind == DFA
    for r in range(8):  # root and skip rows: the first byte of every chunk
        for b in range(1, 256, 2):
            table[r * 256 + b] = 8 << 10
    t = DecodeTable(torch.from_numpy(table.view(np.int32)).to(cuda_device), DFA)
    got = decode(d["luts"], d["encoded"], d["packed_other_4bits"], d["output_positions"],
                 d["gaps"], table=t)
    torch.cuda.synchronize()
    assert np.array_equal(got.view(torch.uint8).cpu().numpy(), flat)


# ---------------------------------------------------------------- edge cases


@pytest.mark.parametrize("kind", [MULTI, DFA])
def test_outputs_past_n_elements_are_untouched(kind, cuda_device):
    flat = _random_block(4)
    block = _compress(flat)
    out = torch.full((flat.size + 64,), 0xAB, dtype=torch.uint8, device=cuda_device)
    got = _gpu_decode(block, cuda_device, n_elements=flat.size, out=out, kind=kind)
    assert np.array_equal(got[: flat.size], flat)
    assert (got[flat.size:] == 0xAB).all()


@pytest.mark.parametrize("kind", [MULTI, DFA])
def test_shorter_n_elements_clamps_like_the_reference(kind, cuda_device):
    flat = _random_block(9)
    block = _compress(flat)
    out = torch.full((flat.size,), 0xCD, dtype=torch.uint8, device=cuda_device)
    n = (flat.size // 3) & ~1
    got = _gpu_decode(block, cuda_device, n_elements=n, out=out, kind=kind)
    assert np.array_equal(got[:n], flat[:n])
    assert (got[n:] == 0xCD).all()


def test_misaligned_output_is_rejected(cuda_device):
    from ecf8_amd.decode import ECF8Error, decode_into

    flat = _random_block(3)
    d = _dev_block(_compress(flat), cuda_device)
    buf = torch.empty(flat.size + 16, dtype=torch.uint8, device=cuda_device)
    with pytest.raises(ECF8Error):
        decode_into(buf[1:1 + flat.size], d["luts"], d["encoded"], d["packed_other_4bits"],
                    d["output_positions"], d["gaps"])


def test_decode_on_a_side_stream(cuda_device):
    from ecf8_amd.decode import decode_into

    flat = _random_block(14)
    d = _dev_block(_compress(flat), cuda_device)
    out = torch.empty(flat.size, dtype=torch.uint8, device=cuda_device)
    s = torch.cuda.Stream(device=cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(s):
        decode_into(out, d["luts"], d["encoded"], d["packed_other_4bits"], d["output_positions"],
                    d["gaps"])
    s.synchronize()
    assert np.array_equal(out.cpu().numpy(), flat)


@pytest.mark.parametrize("seed", [1, 6, 11])  # geometric exponents: 1-bit codes
def test_min_code_bits_unknown_equals_derived(seed, cuda_device):
    from ecf8_amd.decode import decode, min_code_bits

    _say(f"min_code_bits seed {seed}")
    from dfloat.compress import compress_flat

    flat = _random_block(seed)
    res = compress_flat(torch.from_numpy(flat).view(torch.float8_e4m3fn))
    shortest = min(bits for sym, (bits, _) in res["table"].items() if isinstance(sym, int))
    assert min_code_bits(res["luts"]) == shortest
    d = _dev_block({k: res[k] for k in KEYS}, cuda_device)
    table = _table_for(d, MULTI)  # min_code_bits sizes the multi kernel's runs
    for bits in (0, None):
        got = decode(d["luts"], d["encoded"], d["packed_other_4bits"], d["output_positions"],
                     d["gaps"], table=table, min_code_bits=bits)
        torch.cuda.synchronize()
        assert np.array_equal(got.view(torch.uint8).cpu().numpy(), flat)


def test_min_code_bits_above_the_truth_stays_in_bounds(cuda_device):
    """A min_code_bits larger than the block's shortest code sizes the LDS
    runs too small; the kernel clamps its run indexes, so outputs may be
    wrong but nothing outside [0, n) is written."""
    from ecf8_amd.decode import decode_into

    g = dict(np.load(os.path.join(GOLDEN, "single_exponent.npz")))  # 1-bit codes
    n = int(g["flat"].size)
    d = _dev_block(g, cuda_device)
    out = torch.full((n + 256,), 0x5A, dtype=torch.uint8, device=cuda_device)
    table = _table_for(d, MULTI)
    decode_into(out[:n], d["luts"], d["encoded"], d["packed_other_4bits"],
                d["output_positions"], d["gaps"], table=table, min_code_bits=16)
    torch.cuda.synchronize()
    assert (out[n:].cpu().numpy() == 0x5A).all()
    decode_into(out[:n], d["luts"], d["encoded"], d["packed_other_4bits"],
                d["output_positions"], d["gaps"], table=table, min_code_bits=1)
    torch.cuda.synchronize()
    assert np.array_equal(out[:n].cpu().numpy(), g["flat"])


# ------------------------------------------------------- drop-in call forms


@pytest.mark.parametrize("seed", [20, 21])
def test_reference_call_form_of_decode(seed, cuda_device):
    """_decode(grid=, block=, shared_mem=, args=[...]) exactly as
    scripts/compress.py:109-124 calls the CUDA kernel; seed 21 draws a
    geometric histogram with a 1-bit code (the multi-symbol kernel)."""
    from dfloat.run.run import _decode

    flat = _random_block(seed)
    d = _dev_block(_compress(flat), cuda_device)
    n_bytes = d["encoded"].numel()
    op = d["output_positions"].view(torch.uint64).cpu().numpy().astype(np.int64)
    shared = 512 * 4 + 4 + int((op[1:] - op[:-1]).max())
    out = torch.empty(flat.size, dtype=torch.float8_e4m3fn, device=cuda_device)
    _decode(grid=(int(np.ceil(n_bytes / (512 * 8))),), block=(512,), shared_mem=shared,
            args=[d["luts"].data_ptr(), d["encoded"].data_ptr(), d["packed_other_4bits"].data_ptr(),
                  d["output_positions"].data_ptr(), d["gaps"].data_ptr(), out.data_ptr(),
                  d["luts"].shape[0], n_bytes, flat.size])
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.uint8).cpu().numpy(), flat)


def _lut_stacks():
    """LUT stacks of every kind: the golden fixtures, random codes (with and
    without 1-bit codes, long codes), and random bytes (malformed stacks)."""
    stacks = [np.load(os.path.join(GOLDEN, f"{c}.npz"))["luts"] for c in CASES]
    for seed in range(60):
        flat = _random_block(1000 + seed)
        stacks.append(oc.compress_block(flat, 8, 512)["luts"])
    rng = np.random.default_rng(5)
    for _ in range(40):
        stacks.append(rng.integers(0, 256, (int(rng.integers(2, 19)), 256), dtype=np.uint8))
    return stacks


def test_device_table_builder_writes_the_host_builders_bytes(cuda_device):
    """ecf8_build_table (one workgroup on the device) and
    ecf8_build_table_host run the same steps: for every LUT stack and every
    requested kind they write the same ECF8_TABLE_BYTES, kind word included,
    and refuse the automaton for the same stacks."""
    from ecf8_amd.decode import ECF8Error, build_table, build_table_host

    stacks = _lut_stacks()
    _say(f"device table builder: {len(stacks)} LUT stacks")
    n_dfa = 0
    for i, luts in enumerate(stacks):
        d = torch.from_numpy(np.ascontiguousarray(luts)).to(cuda_device)
        for kind in (ANY, MULTI, DFA):
            try:
                want, want_kind = build_table_host(luts, kind)
            except ECF8Error:
                assert kind == DFA
                with pytest.raises(ECF8Error):
                    build_table(d, kind=DFA)
                continue
            got = build_table(d, kind=kind)
            assert got.kind == want_kind, (i, kind)
            assert np.array_equal(got.data.cpu().numpy().view(np.uint32), want), (i, kind)
            if kind == ANY:
                n_dfa += want_kind == DFA
                # asynchronous build: same bytes, kind known on the device only
                lazy = build_table(d, kind=ANY, sync=False)
                assert lazy.kind == ANY
                torch.cuda.synchronize()
                assert np.array_equal(lazy.data.cpu().numpy().view(np.uint32), want), i
    assert n_dfa >= 20  # both kinds are exercised


def test_cached_table_is_rebuilt_only_when_the_luts_change(cuda_device):
    """ecf8_build_table_cached: a zero-filled cache gets the table
    ecf8_build_table writes; a call with unchanged LUTs leaves the cached
    table as it is (a word planted in it survives); a call after the LUT
    bytes (or their row count) change rebuilds it for the new LUTs."""
    from ecf8_amd._lib import ECF8_MAX_LUTS, ECF8_TABLE_BYTES, ECF8_TABLE_CACHE_BYTES, lib
    from ecf8_amd.decode import build_table_host

    stacks = _lut_stacks()[:40]
    L = lib()
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    words = ECF8_TABLE_BYTES // 4
    cache = torch.zeros(ECF8_TABLE_CACHE_BYTES // 8, dtype=torch.int64, device=cuda_device)
    luts_buf = torch.zeros(ECF8_MAX_LUTS * 256, dtype=torch.uint8, device=cuda_device)
    table_of = lambda: cache.view(torch.int32)[:words].cpu().numpy().view(np.uint32)  # noqa: E731
    prev = None
    for i, luts in enumerate(stacks):
        n_luts = luts.shape[0]
        luts_buf[: n_luts * 256].copy_(torch.from_numpy(np.ascontiguousarray(luts).reshape(-1)))
        want, _ = build_table_host(luts, ANY)
        assert L.ecf8_build_table_cached(luts_buf.data_ptr(), n_luts, ANY, cache.data_ptr(),
                                         stream) == 0
        assert np.array_equal(table_of(), want), i
        if prev is not None and np.array_equal(prev, want):
            continue
        # unchanged LUTs: the planted word stays, nothing is rebuilt
        cache.view(torch.int32)[7] = 0x1234567
        assert L.ecf8_build_table_cached(luts_buf.data_ptr(), n_luts, ANY, cache.data_ptr(),
                                         stream) == 0
        got = table_of()
        assert got[7] == 0x1234567 and np.array_equal(np.delete(got, 7), np.delete(want, 7)), i
        prev = want
    # the same bytes under another row count are other LUTs
    n_luts = stacks[-1].shape[0]
    if n_luts > 2:
        cache.view(torch.int32)[7] = 0x1234567
        assert L.ecf8_build_table_cached(luts_buf.data_ptr(), n_luts - 1, ANY, cache.data_ptr(),
                                         stream) == 0
        want, _ = build_table_host(np.ascontiguousarray(stacks[-1][: n_luts - 1]), ANY)
        assert np.array_equal(table_of(), want)
    # refusals on the host, before any launch
    assert L.ecf8_build_table_cached(luts_buf.data_ptr(), 1, ANY, cache.data_ptr(), stream) != 0
    assert L.ecf8_build_table_cached(luts_buf.data_ptr(), 3, DFA, cache.data_ptr(), stream) != 0
    assert L.ecf8_build_table_cached(luts_buf.data_ptr(), 3, ANY, cache.data_ptr() + 4,
                                     stream) != 0


def test_reference_call_form_keeps_one_table_per_lut_buffer(cuda_device):
    """Repeated _decode calls on one block reuse one table cache (no
    allocation after the first call), and the cache count stays bounded."""
    from dfloat.run.run import _decode

    flat = _random_block(3)
    d = _dev_block(_compress(flat), cuda_device)
    n_bytes = d["encoded"].numel()
    out = torch.empty(flat.size, dtype=torch.float8_e4m3fn, device=cuda_device)
    call = dict(grid=(-(-n_bytes // 4096),), block=(512,), shared_mem=0,
                args=[d["luts"].data_ptr(), d["encoded"].data_ptr(),
                      d["packed_other_4bits"].data_ptr(), d["output_positions"].data_ptr(),
                      d["gaps"].data_ptr(), out.data_ptr(), d["luts"].shape[0], n_bytes,
                      flat.size])
    _decode.clear()
    _decode(**call)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(cuda_device)
    for _ in range(5):
        out.view(torch.uint8).zero_()
        _decode(**call)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(cuda_device) == before
    assert len(_decode._caches) == 1
    assert np.array_equal(out.view(torch.uint8).cpu().numpy(), flat)
    old = _decode.max_cached
    copies = [d["luts"].clone() for _ in range(6)]  # six LUT buffers: six cache keys
    try:
        _decode.max_cached = 3
        for luts in copies:
            out.view(torch.uint8).zero_()
            _decode(**dict(call, args=[luts.data_ptr()] + call["args"][1:]))
            assert len(_decode._caches) <= 3
        torch.cuda.synchronize()
        assert np.array_equal(out.view(torch.uint8).cpu().numpy(), flat)
    finally:
        _decode.max_cached = old
        _decode.clear()


@pytest.mark.parametrize("seed", [0, 1, 4, 6])
def test_decode_with_the_kind_read_on_the_device(seed, cuda_device):
    """A table built asynchronously (kind ECF8_TABLE_ANY): the decode
    launches both kernels and the one the table is not for exits; the output
    is bit-exact for automaton and multi-symbol blocks alike."""
    from ecf8_amd.decode import build_table, decode_into

    flat = _random_block(seed)
    d = _dev_block(_compress(flat), cuda_device)
    table = build_table(d["luts"], sync=False)
    out = torch.full((flat.size + 64,), 0x5A, dtype=torch.uint8, device=cuda_device)
    decode_into(out, d["luts"], d["encoded"], d["packed_other_4bits"], d["output_positions"],
                d["gaps"], table=table, n_elements=flat.size)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got[: flat.size], flat)
    assert (got[flat.size:] == 0x5A).all()


def _relabel(flat, perm):
    """The same block with exponent e replaced by perm[e]: the same count
    multiset, so the same bitstream size, under a different code table."""
    e = (flat >> 3) & 0xF
    return ((flat & 0x87) | (perm[e].astype(np.uint8) << 3)).astype(np.uint8)


def test_reference_call_form_is_graph_capturable(cuda_device):
    """_decode in the reference's call form is asynchronous: captured once
    in a HIP graph, then replayed with new contents in the same buffers --
    the same LUTs with a shuffled block, and other LUTs (exponents
    relabelled) -- each replay bit-exact.  A 1-bit code (multi-symbol
    kernel) is among the relabellings."""
    from dfloat.run.run import _decode

    rng = np.random.default_rng(11)
    n = 200_000
    syms = np.array([9, 10, 11, 12, 13, 14, 15, 8, 7, 6, 5, 0])
    p = np.array([0.03, 0.06, 0.11, 0.21, 0.31, 0.23, 0.025, 0.01, 0.004, 0.001, 5e-4, 5e-5])
    exps = rng.choice(syms, n, p=p / p.sum()).astype(np.uint8)
    other = rng.integers(0, 16, n, dtype=np.uint8)
    base = (((other & 8) << 4) | (exps << 3) | (other & 7)).astype(np.uint8)
    variants = [base, rng.permutation(base)]
    for s in range(40):  # relabellings whose LUT stack has the same number of rows
        perm = np.random.default_rng(100 + s).permutation(16)
        v = _relabel(base, perm)
        if _compress(v)["luts"].shape == _compress(base)["luts"].shape:
            variants.append(v)
        if len(variants) == 5:
            break
    blocks = [_compress(v) for v in variants]
    n_bytes = blocks[0]["encoded"].numel()
    assert all(b["encoded"].numel() == n_bytes for b in blocks)
    assert any(not torch.equal(b["luts"], blocks[0]["luts"]) for b in blocks)
    d = _dev_block(blocks[0], cuda_device)
    largest = max(int(np.diff(b["output_positions"].numpy().view(np.uint64).astype(np.int64)).max())
                  for b in blocks)
    out = torch.empty(n, dtype=torch.float8_e4m3fn, device=cuda_device)
    call = dict(grid=(-(-n_bytes // 4096),), block=(512,), shared_mem=512 * 4 + 4 + largest,
                args=[d["luts"].data_ptr(), d["encoded"].data_ptr(),
                      d["packed_other_4bits"].data_ptr(), d["output_positions"].data_ptr(),
                      d["gaps"].data_ptr(), out.data_ptr(), d["luts"].shape[0], n_bytes, n])
    side = torch.cuda.Stream(cuda_device)
    side.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(side):
        _decode(**call)  # warm-up outside the capture
    torch.cuda.current_stream(cuda_device).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _decode(**call)
    _say(f"graph-captured _decode: {len(blocks)} variants")
    for rep in range(2):
        for i, (flat, b) in enumerate(zip(variants, blocks)):
            for k in KEYS:
                d[k].copy_(b[k].contiguous().view(torch.uint8))
            out.view(torch.uint8).fill_(0)
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.view(torch.uint8).cpu().numpy(), flat), (rep, i)


def test_validate_cuda_decoding_fp8_api(cuda_device):
    from dfloat.compress import compress_flat, validate_cuda_decoding_fp8

    flat = torch.from_numpy(_random_block(4)).view(torch.float8_e4m3fn)
    res = compress_flat(flat)
    validate_cuda_decoding_fp8({"threads_per_block": 512, "bytes_per_thread": 8}, res, cuda_device)


class _Block(nn.Module):
    def __init__(self, shapes):
        super().__init__()
        self.attn = nn.Module()
        self.mlp = nn.Module()
        for path, (o, i) in shapes.items():
            parent, name = path.split(".")
            setattr(getattr(self, parent), name, nn.Linear(i, o, bias=False))

    def forward(self, x):
        return x


def test_forward_pre_hook_injects_bit_exact_weights(cuda_device):
    """Block-level hook flow: flatten name-sorted linears, compress, register
    buffers + hook the way the loader does (run.py:406-458), forward, and
    compare every injected .weight with the original FP8 tensor."""
    from dfloat.compress import compress_flat
    from dfloat.run.run import TensorManager, _process_compressed_tensor
    from ecf8_amd.synth import synthetic_fp8
    from dfloat.utils import flatten_block_of_weights

    shapes = {"attn.q": (256, 128), "attn.k": (128, 128), "mlp.up": (384, 128)}
    blk = _Block(shapes)
    orig = {}
    for i, (path, (o, inp)) in enumerate(sorted(shapes.items())):
        w, _ = synthetic_fp8(o, inp, 0.02, seed=i)
        lin = blk.get_submodule(path)
        lin.weight = nn.Parameter(w, requires_grad=False)
        orig[path] = w.view(torch.uint8).clone()
    layers = {p: blk.get_submodule(p) for p in sorted(shapes)}
    flat, split = flatten_block_of_weights(layers)
    res = compress_flat(flat)
    pattern = {r"block": sorted(shapes)}
    for key in ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps"):
        _process_compressed_tensor(blk, key, res[key], f"block.{key}", pattern, 512, 8)
    _process_compressed_tensor(blk, "split_positions", split, "block.split_positions", pattern,
                               512, 8)
    for path in shapes:
        assert "weight" not in blk.get_submodule(path)._parameters
    blk.to(cuda_device)
    TensorManager.clear_device()
    blk(torch.zeros(1, device=cuda_device))
    torch.cuda.synchronize()
    for path in shapes:
        w = blk.get_submodule(path).weight
        assert w.dtype == torch.float8_e4m3fn and tuple(w.shape) == shapes[path]
        assert torch.equal(w.view(torch.uint8).cpu(), orig[path])

    # later calls take the prepared launch: the shared buffer overwritten in
    # between is decoded again, and a view replaced in between is injected
    # again
    buf = TensorManager.get_tensor(cuda_device, flat.numel())
    views = {p: blk.get_submodule(p).weight for p in shapes}
    for rep in range(3):
        buf.view(torch.uint8).fill_(0x3C)
        if rep == 2:
            blk.get_submodule("attn.k").weight = torch.zeros(1, device=cuda_device)
        blk(torch.zeros(1, device=cuda_device))
        torch.cuda.synchronize()
        for path in shapes:
            w = blk.get_submodule(path).weight
            if rep < 2:  # nothing replaced: the same views
                assert w is views[path]
            assert w.dtype == torch.float8_e4m3fn and tuple(w.shape) == shapes[path]
            assert torch.equal(w.view(torch.uint8).cpu(), orig[path]), (rep, path)


# ---------------------------------------------------------- batched launch


def _batched_case(blocks_flat, cuda_device, blocks_per_task):
    from ecf8_amd.decode import build_table, decode_batched

    blocks, bufs, tables = [], [], []
    for flat in blocks_flat:
        d = _dev_block(_compress(flat), cuda_device)
        blocks.append(d)
        tables.append(build_table(d["luts"]))
        bufs.append(torch.full((flat.size + 32,), 0x3C, dtype=torch.uint8, device=cuda_device))
    decode_batched(blocks, [b[: f.size] for b, f in zip(bufs, blocks_flat)], tables,
                   blocks_per_task=blocks_per_task)
    torch.cuda.synchronize()
    for i, (buf, flat) in enumerate(zip(bufs, blocks_flat)):
        got = buf.cpu().numpy()
        assert np.array_equal(got[: flat.size], flat), f"block {i}"
        assert (got[flat.size:] == 0x3C).all(), f"block {i} wrote past its end"
    return tables


@pytest.mark.parametrize("blocks_per_task", [1, 3, 16, 100000])
def test_batched_decode_of_mixed_blocks(blocks_per_task, cuda_device):
    """Random blocks of every distribution kind and size (some only the
    multi-symbol table can decode, some too small to batch) in one call."""
    _say(f"batched mixed blocks_per_task={blocks_per_task}")
    flats = [_random_block(s) for s in range(30, 42)]
    flats.append(np.array([0x41, 0xC2], np.uint8))  # a two-element block
    tables = _batched_case(flats, cuda_device, blocks_per_task)
    assert {t.kind for t in tables} == {MULTI, DFA}


def test_batched_decode_of_moe_experts(cuda_device):
    """An MoE layer's attention block and 16 experts (the reference
    compresses each expert as its own block) in one launch."""
    from ecf8_amd import synth

    _say("batched moe experts")
    flats = [synth.flat_block(synth.synthetic_block(synth.QWEN3_MOE_ATTN, 0))[0]]
    flats += [synth.flat_block(synth.synthetic_block(synth.QWEN3_MOE_EXPERT, 1 + e))[0]
              for e in range(16)]
    _batched_case([f.view(torch.uint8).numpy() for f in flats], cuda_device, 16)


def _select_case(cuda_device, n_experts=12, blocks_per_task=4):
    """An attention block and n_experts small expert blocks (all automaton
    tables), outputs filled with a sentinel."""
    from ecf8_amd import synth
    from ecf8_amd.decode import BatchSelect, build_table, prepare_batch

    shapes = {"down_proj": (256, 384, 0.02), "gate_proj": (384, 256, 0.02),
              "up_proj": (384, 256, 0.02)}
    flats = [synth.flat_block(synth.synthetic_block(synth.QWEN3_MOE_ATTN, 0))[0]]
    flats += [synth.flat_block(synth.synthetic_block(shapes, 10 + e))[0] for e in range(n_experts)]
    flats = [f.view(torch.uint8).numpy() for f in flats]
    blocks = [_dev_block(_compress(f), cuda_device) for f in flats]
    tables = [build_table(b["luts"]) for b in blocks]
    assert all(t.kind == DFA for t in tables)
    bufs = [torch.full((f.size + 32,), 0x3C, dtype=torch.uint8, device=cuda_device) for f in flats]
    plan = prepare_batch(blocks, [b[: f.size] for b, f in zip(bufs, flats)], tables,
                         blocks_per_task=blocks_per_task)
    return flats, bufs, BatchSelect(plan)


def _check_selected(flats, bufs, flags):
    for i, (buf, flat) in enumerate(zip(bufs, flats)):
        got = buf.cpu().numpy()
        if flags[i]:
            assert np.array_equal(got[: flat.size], flat), f"selected block {i}"
        else:
            assert (got[: flat.size] == 0x3C).all(), f"unselected block {i} was written"
        assert (got[flat.size:] == 0x3C).all(), f"block {i} wrote past its end"


def test_batched_select_decodes_only_the_selected_blocks(cuda_device):
    """ecf8_decode_batched_select: the attention block plus a random subset
    of experts per call (flags on the device), several selections in a row,
    none and all included."""
    _say("batched select")
    flats, bufs, sel = _select_case(cuda_device)
    rng = np.random.default_rng(3)
    cases = [np.ones(len(flats), np.int32), np.zeros(len(flats), np.int32)]
    for _ in range(4):
        f = (rng.random(len(flats)) < 0.5).astype(np.int32)
        f[0] = 1
        cases.append(f)
    for flags in cases:
        for b in bufs:
            b.fill_(0x3C)
        sel(torch.from_numpy(flags).to(cuda_device))
        torch.cuda.synchronize()
        _check_selected(flats, bufs, flags)
        n_sel, n_tasks = sel.counts.cpu().tolist()
        assert n_sel == int(flags.sum())
        assert n_tasks == _selected_tasks(sel.plan, flags)


def _selected_tasks(plan, flags):
    """Tasks of the selected descriptors (flags per descriptor)."""
    from ecf8_amd.decode import BLOCK_DESC_DTYPE

    n_bytes = np.frombuffer(plan.descs.cpu().numpy().tobytes(), dtype=BLOCK_DESC_DTYPE)["n_bytes"]
    fb = -(-n_bytes // (plan.threads_per_block * 8))
    tasks = -(-fb // plan.blocks_per_task)
    return int(tasks[np.asarray(flags)[: plan.count] != 0].sum())


def test_batched_select_replays_in_a_graph_with_new_flags(cuda_device):
    """The select call captured once in a HIP graph decodes whatever the
    flags tensor holds at each replay (eager work between replays)."""
    _say("batched select graph")
    flats, bufs, sel = _select_case(cuda_device, n_experts=8)
    flags_dev = torch.zeros(len(flats), dtype=torch.int32, device=cuda_device)
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(s):
        sel(flags_dev)  # warm-up (launch caches)
    torch.cuda.current_stream(cuda_device).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sel(flags_dev)
    rng = np.random.default_rng(5)
    for _ in range(3):
        f = (rng.random(len(flats)) < 0.5).astype(np.int32)
        f[0] = 1
        for b in bufs:
            b.fill_(0x3C)
        flags_dev.copy_(torch.from_numpy(f).to(cuda_device))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _check_selected(flats, bufs, f)


def test_batched_select_with_blocks_outside_the_batched_kernel(cuda_device):
    """Flags are per block in the order given to prepare_batch, also when
    some blocks (a multi-symbol table, a tiny block) are not in the batched
    launch: the batched blocks follow their flags, the others are decoded on
    every call.  Eager and graph-replayed."""
    from ecf8_amd.decode import BatchSelect, build_table, prepare_batch

    _say("batched select with singles")
    flats = [_random_block(s) for s in (30, 31, 32, 33, 34, 35, 36, 37, 39, 44, 49)]
    flats.insert(3, np.array([0x41, 0xC2, 0x33, 0x0A], np.uint8))  # too small to batch
    blocks = [_dev_block(_compress(f), cuda_device) for f in flats]
    tables = [build_table(b["luts"]) for b in blocks]
    bufs = [torch.full((f.size + 32,), 0x3C, dtype=torch.uint8, device=cuda_device) for f in flats]
    plan = prepare_batch(blocks, [b[: f.size] for b, f in zip(bufs, flats)], tables,
                         blocks_per_task=2)
    single = [i for i in range(len(flats)) if i not in plan.desc_blocks]
    assert plan.singles and plan.count and 3 in single
    assert any(tables[i].kind == MULTI for i in single)
    sel = BatchSelect(plan)
    flags_dev = torch.zeros(len(flats), dtype=torch.int32, device=cuda_device)

    def check(f):
        for i, (buf, flat) in enumerate(zip(bufs, flats)):
            got = buf.cpu().numpy()
            if f[i] or i in single:
                assert np.array_equal(got[: flat.size], flat), f"block {i}"
            else:
                assert (got[: flat.size] == 0x3C).all(), f"unselected block {i} was written"
            assert (got[flat.size:] == 0x3C).all(), f"block {i} wrote past its end"

    rng = np.random.default_rng(8)
    draws = [(rng.random(len(flats)) < 0.5).astype(np.int32) for _ in range(3)]
    for f in draws:
        for b in bufs:
            b.fill_(0x3C)
        flags_dev.copy_(torch.from_numpy(f).to(cuda_device))
        sel(flags_dev)
        torch.cuda.synchronize()
        check(f)
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(s):
        sel(flags_dev)
    torch.cuda.current_stream(cuda_device).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sel(flags_dev)
    for f in draws[::-1]:
        for b in bufs:
            b.fill_(0x3C)
        flags_dev.copy_(torch.from_numpy(f).to(cuda_device))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(f)


def _many_blocks(cuda_device, n, tpb=512):
    """n small blocks (one or two 128 x 128 Linears: 2 or 3 format-blocks
    each at 512 threads per block), all automaton tables, outputs filled
    with a sentinel."""
    from ecf8_amd import synth

    one = {"up_proj": (128, 128, 0.02)}
    two = {"down_proj": (128, 128, 0.02), "up_proj": (128, 128, 0.02)}
    flats = [synth.flat_block(synth.synthetic_block(two if e % 3 else one, 500 + e))[0]
             .view(torch.uint8).numpy() for e in range(n)]
    blocks = [_dev_block(_compress(f, tpb), cuda_device) for f in flats]
    bufs = [torch.full((f.size + 32,), 0x3C, dtype=torch.uint8, device=cuda_device) for f in flats]
    return flats, blocks, bufs


@pytest.mark.parametrize("n_blocks", [256, 264])
def test_batched_launch_on_either_side_of_the_lds_task_table(n_blocks, cuda_device):
    """A routed launch of up to 256 descriptors selects in the batched
    kernel itself (each workgroup scans the flags and task counts into an
    LDS task table); above, a compaction kernel runs first.  Whole launches
    search the descriptors in memory.  Every path bit-exact, unselected
    outputs untouched, the counts written, eager and replayed in a graph."""
    from ecf8_amd.decode import BatchSelect, build_table, prepare_batch

    _say(f"batched over {n_blocks} blocks")
    flats, blocks, bufs = _many_blocks(cuda_device, n_blocks)
    tables = [build_table(b["luts"]) for b in blocks]
    assert all(t.kind == DFA for t in tables)
    plan = prepare_batch(blocks, [b[: f.size] for b, f in zip(bufs, flats)], tables,
                         blocks_per_task=2)
    assert plan.count == n_blocks and not plan.singles
    from ecf8_amd.decode import decode_batched

    decode_batched(blocks, [b[: f.size] for b, f in zip(bufs, flats)], tables, blocks_per_task=2)
    torch.cuda.synchronize()
    _check_selected(flats, bufs, np.ones(n_blocks, np.int32))

    sel = BatchSelect(plan)
    flags_dev = torch.zeros(n_blocks, dtype=torch.int32, device=cuda_device)
    rng = np.random.default_rng(n_blocks)
    draws = [(rng.random(n_blocks) < p).astype(np.int32) for p in (0.5, 0.1, 0.9)]
    for f in draws:
        for b in bufs:
            b.fill_(0x3C)
        flags_dev.copy_(torch.from_numpy(f).to(cuda_device))
        sel(flags_dev)
        torch.cuda.synchronize()
        _check_selected(flats, bufs, f)
        assert sel.counts.cpu().tolist() == [int(f.sum()), _selected_tasks(plan, f)]
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(s):
        sel(flags_dev)
    torch.cuda.current_stream(cuda_device).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sel(flags_dev)
    for f in draws[::-1]:
        for b in bufs:
            b.fill_(0x3C)
        flags_dev.copy_(torch.from_numpy(f).to(cuda_device))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _check_selected(flats, bufs, f)


@pytest.mark.parametrize("tpb,n_blocks", [(128, 200), (256, 40), (1024, 40)])
def test_batched_launch_at_every_block_size(tpb, n_blocks, cuda_device):
    """The batched kernel at 128, 256 and 1024 threads per format-block (the
    other format geometries; 128 threads scan the LDS task table in two
    passes): whole and routed launches bit-exact, unselected outputs
    untouched, the routed counts written."""
    from ecf8_amd.decode import BatchSelect, build_table, decode_batched, prepare_batch

    _say(f"batched at tpb={tpb} over {n_blocks} blocks")
    flats, blocks, bufs = _many_blocks(cuda_device, n_blocks, tpb)
    tables = [build_table(b["luts"]) for b in blocks]
    assert all(t.kind == DFA for t in tables)
    outs = [b[: f.size] for b, f in zip(bufs, flats)]
    plan = prepare_batch(blocks, outs, tables, threads_per_block=tpb, blocks_per_task=2)
    assert plan.count == n_blocks and not plan.singles
    decode_batched(plan)
    torch.cuda.synchronize()
    _check_selected(flats, bufs, np.ones(n_blocks, np.int32))
    sel = BatchSelect(plan)
    rng = np.random.default_rng(tpb)
    for p in (0.5, 0.2):
        f = (rng.random(n_blocks) < p).astype(np.int32)
        for b in bufs:
            b.fill_(0x3C)
        sel(torch.from_numpy(f).to(cuda_device))
        torch.cuda.synchronize()
        _check_selected(flats, bufs, f)
        assert sel.counts.cpu().tolist() == [int(f.sum()), _selected_tasks(plan, f)]
