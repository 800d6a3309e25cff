"""Derived decode tables (ecf8_amd/csrc/ecf8_tables.cpp), checked on the CPU
against the oracle's statement of the reference decode rule
(dfloat/run/decode.cu:85-112): the multi-symbol table entry by entry, and the
byte automaton by walking it over every chunk of real compressed blocks
exactly as the DFA kernel does, comparing each chunk's symbols with the
oracle's."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import codec as oc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
CASES = sorted(json.load(open(os.path.join(GOLDEN, "index.json"))))

ROW_MASK = 0x7C00
EXACT_ROW = 8
FIRST_PENDING_ROW = 9
SKIP_BYTE = 24 * 256


def _golden(name):
    return dict(np.load(os.path.join(GOLDEN, f"{name}.npz")))


def _table(luts, kind):
    from ecf8_amd.decode import build_table_host

    return build_table_host(luts, kind)


def _dfa_chunk_symbols(table, enc, gaps, g):
    """Step 1 of decode_dfa_kernel for chunk g: 8 byte lookups from the
    row for the chunk's gap, then the code open at bit 64 (if any) from the
    look-ahead bytes."""
    b = [int(enc[8 * g + i]) if 8 * g + i < enc.size else 0 for i in range(10)]
    gb = int(gaps[g // 2])
    gap = (gb >> 4) if g % 2 == 0 else gb & 0xF
    off = (gap << 10) | (b[0] << 2) if gap < 8 else SKIP_BYTE * 4 + ((gap - 8) << 2)
    entries = [int(table[off >> 2])]
    for k in range(1, 8):
        entries.append(int(table[((entries[-1] & ROW_MASK) | (b[k] << 2)) >> 2]))
    row7 = entries[-1] & ROW_MASK
    if row7 == EXACT_ROW << 10:
        return None  # the kernel decodes this chunk with the LUT rule itself
    is_open = row7 >= FIRST_PENDING_ROW << 10
    e8 = int(table[(row7 | (b[8] << 2)) >> 2])
    if is_open and (e8 & 0xFF) == 0:
        e8 = int(table[((e8 & ROW_MASK) | (b[9] << 2)) >> 2])
    syms = []
    for e in entries:
        n = (e & 0xFF) >> 2
        assert e & 0xFF == 4 * n
        syms += [(e >> (16 + 4 * i)) & 0xF for i in range(n)]
        assert e >> (16 + 4 * n) == 0  # unused nibbles are zero
    if is_open:
        syms.append((e8 >> 16) & 0xF)
    return syms


def _check_dfa_block(luts, enc, gaps):
    from ecf8_amd.decode import ECF8_TABLE_DFA

    table, kind = _table(luts, ECF8_TABLE_DFA)
    assert kind == ECF8_TABLE_DFA
    n_chunks = -(-enc.size // 8)
    for g in range(n_chunks):
        want = oc.decode_chunk_symbols(luts, enc, gaps, g)
        got = _dfa_chunk_symbols(table, enc, gaps, g)
        if got is None:
            # only the EOF padding of the stream's last chunk leads there
            assert g == n_chunks - 1, f"chunk {g} of {n_chunks} left the automaton"
            continue
        assert got == want, f"chunk {g}"


def _random_block_min_len2(rng):
    """A random compressed block whose Huffman code has no 1-bit code (what
    the automaton requires), drawn until one qualifies."""
    while True:
        k = int(rng.integers(3, 17))
        syms = rng.choice(16, k, replace=False)
        p = rng.pareto(0.3 + 2 * rng.random(), k) + 0.05
        n = int(rng.integers(1000, 20000)) * 2
        exps = rng.choice(syms, n, p=p / p.sum()).astype(np.uint8)
        other = rng.integers(0, 16, n, dtype=np.uint8)
        flat = (((other & 8) << 4) | (exps << 3) | (other & 7)).astype(np.uint8)
        blk = oc.compress_block(flat, 8, 512)
        lengths = blk["luts"][-1]
        if lengths[lengths > 0].min() >= 2:
            return blk


# ---------------------------------------------------------------- multi


@pytest.mark.parametrize("name", CASES)
def test_multi_table_entries_follow_the_lut_rule(name):
    from ecf8_amd.decode import ECF8_TABLE_MULTI

    luts = _golden(name)["luts"]
    table, kind = _table(luts, ECF8_TABLE_MULTI)
    assert kind == ECF8_TABLE_MULTI
    rng = np.random.default_rng(0)
    for w in range(4096):
        e = int(table[w])
        total = e >> 28
        mask = (e >> 16) & 0xFFF
        n = bin(mask).count("1")
        if total == 0:
            assert e == 0
            continue
        for _ in range(3):
            bits = (w << 20) | int(rng.integers(0, 1 << 20))  # window + any continuation
            off = 0
            for k in range(n):
                assert mask >> off & 1
                sym, ln = oc.lut_decode_one(luts, (bits >> (16 - off)) & 0xFFFF)
                assert sym == (e >> (4 * k)) & 0xF and ln > 0
                off += ln
            assert off == total <= 12


# ------------------------------------------------------------------ dfa


@pytest.mark.parametrize("name", ["synth_128x256", "synth_128x256_tpb128", "uniform_exponents"])
def test_dfa_walk_equals_oracle_on_golden_blocks(name):
    g = _golden(name)
    _check_dfa_block(g["luts"], g["encoded"], g["gaps"])


@pytest.mark.parametrize("seed", range(12))
def test_dfa_walk_equals_oracle_on_random_codes(seed):
    blk = _random_block_min_len2(np.random.default_rng(100 + seed))
    _check_dfa_block(blk["luts"], blk["encoded"], blk["gaps"])


def test_dfa_is_chosen_for_the_synthetic_weight_histogram():
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import ECF8_TABLE_ANY, ECF8_TABLE_DFA
    from ecf8_amd.synth import synthetic_fp8

    w, _ = synthetic_fp8(256, 512, 0.02, seed=3)
    res = compress_flat(w.reshape(-1))
    _, kind = _table(res["luts"], ECF8_TABLE_ANY)
    assert kind == ECF8_TABLE_DFA
    _check_dfa_block(res["luts"].numpy(), res["encoded"].numpy(), res["gaps"].numpy())


@pytest.mark.parametrize("name", ["single_exponent", "fibonacci_long_codes", "two_elements"])
def test_one_bit_codes_fall_back_to_the_multi_table(name):
    """A 1-bit code can complete 5+ codes in one byte: the automaton refuses
    (asked for explicitly) and the builder's own choice is the multi table."""
    from ecf8_amd.decode import ECF8_TABLE_ANY, ECF8_TABLE_DFA, ECF8_TABLE_MULTI, ECF8Error

    luts = _golden(name)["luts"]
    assert int(luts[-1][luts[-1] > 0].min()) == 1
    with pytest.raises(ECF8Error):
        _table(luts, ECF8_TABLE_DFA)
    _, kind = _table(luts, ECF8_TABLE_ANY)
    assert kind == ECF8_TABLE_MULTI


def test_dfa_rows_stay_inside_the_table():
    from ecf8_amd.decode import ECF8_TABLE_DFA

    table, _ = _table(_golden("synth_128x256")["luts"], ECF8_TABLE_DFA)
    used = table[: SKIP_BYTE + 8]
    assert ((used & ROW_MASK) >> 10).max() < 24
    assert (used & 0xFF).max() <= 16 and ((used & 0xFF) % 4).max() == 0
    assert ((used >> 8) & 3).max() == 0 and ((used >> 15) & 1).max() == 0


def test_corrupt_luts_never_crash_the_builder():
    from ecf8_amd.decode import ECF8_TABLE_ANY

    rng = np.random.default_rng(7)
    for _ in range(20):
        luts = rng.integers(0, 256, (int(rng.integers(2, 19)), 256), dtype=np.uint8)
        table, kind = _table(luts, ECF8_TABLE_ANY)
        assert kind in (0, 1)
        if kind == 1:
            assert ((table[: SKIP_BYTE + 8] & ROW_MASK) >> 10).max() < 24


def test_table_helpers_reject_bad_input():
    from ecf8_amd.decode import ECF8Error

    with pytest.raises(ECF8Error):
        _table(np.zeros((1, 256), np.uint8), -1)
    with pytest.raises(ECF8Error):
        _table(np.zeros((3, 256), np.uint8), 5)
    with pytest.raises(ECF8Error):
        _table(torch.zeros(300, dtype=torch.uint8), -1)
