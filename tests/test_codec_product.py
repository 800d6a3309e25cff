"""The product codec (ecf8_amd.huffman / utils / libecf8 host encoder and
validator) against the oracle and the golden vectors.  CPU only."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import codec as oc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
CASES = sorted(json.load(open(os.path.join(GOLDEN, "index.json"))))


def _golden(name):
    return dict(np.load(os.path.join(GOLDEN, f"{name}.npz")))


def _random_counter(rng):
    k = int(rng.integers(1, 17))
    syms = sorted(rng.choice(16, k, replace=False).tolist())
    counts = (rng.pareto(0.3 + rng.random() * 3, k) * 500 + 1).astype(np.int64)
    if rng.random() < 0.3:  # many ties
        counts = rng.integers(1, 4, k)
    return {int(s): int(c) for s, c in zip(syms, counts)}


@pytest.mark.parametrize("seed", range(200))
def test_huffman_table_equals_restated_dahuffman(seed):
    from dfloat.huffman import HuffmanCodec

    counter = _random_counter(np.random.default_rng(seed))
    ours = HuffmanCodec.from_frequencies(counter).get_code_table()
    ref = oc.HuffmanTable.from_frequencies(counter).get_code_table()
    # same codes in the same listing order (the LUT row order depends on it)
    assert [(repr(k), v) for k, v in ours.items()] == [(repr(k), v) for k, v in ref.items()]


@pytest.mark.parametrize("seed", range(100))
def test_luts_equal_oracle(seed):
    from dfloat.utils import get_luts_from_huffman_table, get_nbit_codec

    counter = _random_counter(np.random.default_rng(1000 + seed))
    table = get_nbit_codec(counter, 16)[2]
    ref_table = oc.get_nbit_codec(counter, 16)[2]
    assert np.array_equal(get_luts_from_huffman_table(table).numpy(),
                          oc.get_luts_from_huffman_table(ref_table))


@pytest.mark.parametrize("name", CASES)
def test_product_compressor_reproduces_golden(name):
    from dfloat.compress import compress_flat

    g = _golden(name)
    tpb = int(g["threads_per_block"])
    flat = torch.from_numpy(g["flat"]).view(torch.float8_e4m3fn)
    res = compress_flat(flat, 8, tpb)
    for key in ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps"):
        assert np.array_equal(res[key].numpy(), g[key]), key


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    g = _golden(name)
    tpb = int(g["threads_per_block"])
    res = oc.compress_block(g["flat"], 8, tpb)
    assert np.array_equal(res["encoded"], g["encoded"])
    assert np.array_equal(res["output_positions"].view(np.uint8), g["output_positions"])
    out = oc.decode(g["luts"], g["encoded"], g["packed_other_4bits"], g["output_positions"],
                    g["gaps"], threads_per_block=tpb)
    assert np.array_equal(out, g["flat"])


@pytest.mark.parametrize("shape", [(4096, 4096), (1000, 2)])
def test_product_encoder_equals_c_oracle_at_size(shape, oracle_native):
    from dfloat.huffman import HuffmanCodec
    from ecf8_amd.synth import synthetic_fp8
    from dfloat.utils import encode_exponents_for_cuda, get_exponents_and_other_4bits_fp8_e4m3

    if shape == (1000, 2):
        w = torch.from_numpy(np.random.default_rng(0).integers(0, 256, 2000, dtype=np.uint8))
        w = w.view(torch.float8_e4m3fn)
    else:
        w = synthetic_fp8(*shape, 0.02, seed=0)[0].reshape(-1)
    exps, _ = get_exponents_and_other_4bits_fp8_e4m3(w.reshape(-1))
    vals, counts = torch.unique(exps, return_counts=True)
    counter = {int(v): int(c) for v, c in zip(vals.tolist(), counts.tolist())}
    codec = HuffmanCodec.from_frequencies(counter)
    enc, gaps, op = encode_exponents_for_cuda(exps, codec)
    ref_codec = oc.HuffmanTable.from_frequencies(counter)
    e2, g2, o2 = oracle_native.encode(exps.numpy(), ref_codec._table, ref_codec._eof)
    assert np.array_equal(enc.numpy(), e2)
    assert np.array_equal(gaps.numpy(), g2)
    assert np.array_equal(op.numpy(), o2)


# ------------------------------------------------------------- validator


def _valid_block():
    g = _golden("synth_128x256")
    return g


def _validate(g, **over):
    from ecf8_amd.decode import validate_format

    args = dict(luts=torch.from_numpy(g["luts"]), encoded_bytes=g["encoded"].size,
                packed_other_4bits_bytes=g["packed_other_4bits"].size,
                output_positions=torch.from_numpy(g["output_positions"]),
                gaps_bytes=g["gaps"].size)
    args.update(over)
    validate_format(**args)


def test_validator_accepts_golden_blocks():
    for name in CASES:
        g = _golden(name)
        _validate(g) if int(g["threads_per_block"]) == 512 else None


@pytest.mark.parametrize("fault", ["truncated_positions", "decreasing_positions", "last_not_n",
                                   "odd_packed", "bad_pointer", "too_many_luts", "gaps_size",
                                   "bad_entry", "first_not_zero"])
def test_validator_rejects_fault(fault):
    from ecf8_amd._lib import ECF8Error

    g = _valid_block()
    op = g["output_positions"].view(np.uint64).copy()
    luts = g["luts"].copy()
    over = {}
    if fault == "truncated_positions":
        over["output_positions"] = torch.from_numpy(op[:-1].view(np.uint8))
    elif fault == "decreasing_positions":
        op[1], op[2] = op[2], op[1]
        over["output_positions"] = torch.from_numpy(op.view(np.uint8))
    elif fault == "last_not_n":
        op[-1] -= 2
        over["output_positions"] = torch.from_numpy(op.view(np.uint8))
    elif fault == "first_not_zero":
        op[0] = 1
        over["output_positions"] = torch.from_numpy(op.view(np.uint8))
    elif fault == "odd_packed":
        over["packed_other_4bits_bytes"] = g["packed_other_4bits"].size - 1
    elif fault == "bad_pointer":
        luts[0, 5] = 256 - (luts.shape[0] - 1)  # points at the length row
        over["luts"] = torch.from_numpy(luts)
    elif fault == "too_many_luts":
        over["luts"] = torch.from_numpy(np.concatenate([luts] * 7))
    elif fault == "gaps_size":
        over["gaps_bytes"] = g["gaps"].size + 1
    elif fault == "bad_entry":
        luts[0, 7] = 100
        over["luts"] = torch.from_numpy(luts)
    with pytest.raises(ECF8Error):
        _validate(g, **over)


def test_encoder_rejects_symbol_without_code():
    from ecf8_amd._lib import ECF8Error
    from dfloat.huffman import HuffmanCodec
    from dfloat.utils import encode_exponents_for_cuda

    codec = HuffmanCodec.from_frequencies({3: 10, 4: 5})
    with pytest.raises(ECF8Error):
        encode_exponents_for_cuda(np.array([3, 4, 5], np.uint8), codec)


def test_product_length_limiter_equals_the_oracle_on_a_large_alphabet():
    """The product's limiter (dfloat/huffman.py, utils.py:249-265) never
    fires for 4-bit exponents: 16 symbols plus EOF are 17 leaves, so no code
    exceeds 16 bits.  It is generic over the alphabet, so it is checked on
    20 Fibonacci-weighted symbols (an unlimited tree 19 deep): same code
    table and same clamped counter as the oracle, longest code <= 16."""
    from dfloat.huffman import HuffmanCodec
    from dfloat.utils import get_nbit_codec

    counts = [1, 1]
    while len(counts) < 20:
        counts.append(counts[-1] + counts[-2])
    counter = {s: c for s, c in enumerate(counts)}
    unlimited = HuffmanCodec.from_frequencies(counter).get_code_table()
    assert max(b for b, _ in unlimited.values()) > 16
    codec, used, table = get_nbit_codec(counter, 16)
    _, ref_used, ref_table = oc.get_nbit_codec(counter, 16)
    assert max(b for b, _ in table.values()) <= 16
    assert {str(k): v for k, v in table.items()} == {str(k): v for k, v in ref_table.items()}
    assert dict(used) == dict(ref_used)
    assert codec.get_code_table() is table
