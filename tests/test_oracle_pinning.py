"""Pins the CPU oracle (oracle/) to facts that do not come from the oracle:
closed forms of the FP8 bit layout, Huffman optimality, brute force over the
code words, bit strings built independently of the streaming encoder, and
round trips to the original bytes (the reference's own check,
scripts/compress.py:126).  CPU only."""

from __future__ import annotations

import heapq
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import codec as oc

# ---------------------------------------------------------------- FP8 split


def test_split_merge_all_bytes_round_trip():
    b = np.arange(256, dtype=np.uint8)
    exps, packed = oc.split_fp8(b)
    assert np.array_equal(oc.merge_fp8(exps, packed), b)


def test_split_matches_e4m3fn_value_decomposition():
    # |value| = 2**(e-7) * (1 + m/8) for e > 0, 2**-6 * m/8 for e == 0; the
    # sign bit is the top bit of the other nibble (NaN = 0x7F/0xFF skipped)
    b = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy()
    exps, packed = oc.split_fp8(b)
    other = np.empty(256, np.uint8)
    other[0::2], other[1::2] = packed >> 4, packed & 0xF
    for i in range(256):
        if np.isnan(vals[i]):
            continue
        e, m, s = int(exps[i]), int(other[i] & 7), int(other[i] >> 3)
        mag = 2.0 ** (e - 7) * (1 + m / 8) if e else 2.0 ** -6 * (m / 8)
        assert (-mag if s else mag) == vals[i] or (mag == 0 and vals[i] == 0)


# ------------------------------------------------------------ Huffman table


def _random_counter(rng, skew):
    k = int(rng.integers(1, 17))
    syms = rng.choice(16, k, replace=False)
    counts = (rng.pareto(skew, k) * 1000 + 1).astype(np.int64)
    return {int(s): int(c) for s, c in zip(sorted(syms), counts[np.argsort(syms)])}


def _textbook_cost(weights):
    h = list(weights)
    heapq.heapify(h)
    cost = 0
    while len(h) > 1:
        a, b = heapq.heappop(h), heapq.heappop(h)
        cost += a + b
        heapq.heappush(h, a + b)
    return cost


@pytest.mark.parametrize("seed", range(40))
def test_huffman_table_is_complete_prefix_free_and_optimal(seed):
    rng = np.random.default_rng(seed)
    counter = _random_counter(rng, 0.5 + (seed % 5))
    codec = oc.HuffmanTable.from_frequencies(counter)
    table = codec.get_code_table()
    assert codec._eof in table and len(table) == len(counter) + 1
    words = [format(v, f"0{b}b") for b, v in table.values()]
    assert all(len(w) == b for w, (b, _) in zip(words, table.values()))
    # Kraft equality: a full binary tree
    assert sum(2.0 ** -b for b, _ in table.values()) == 1.0
    # prefix-free
    for a, b in itertools.permutations(words, 2):
        assert not b.startswith(a)
    # optimal weighted length (EOF has weight 1)
    weights = dict(counter)
    cost = sum(weights.get(s, 1) * b for s, (b, _) in table.items())
    assert cost == _textbook_cost(list(counter.values()) + [1])


def test_sixteen_exponents_never_need_the_length_limiter():
    # 16 symbols + EOF = 17 leaves: no code can be longer than 16 bits, the
    # worst case being the Fibonacci caterpillar
    counts = [1, 1]
    while len(counts) < 16:
        counts.append(counts[-1] + counts[-2])
    table = oc.HuffmanTable.from_frequencies({s: c for s, c in enumerate(counts)}).get_code_table()
    assert max(b for b, _ in table.values()) == 16


def test_length_limiter_caps_codes_at_16_bits():
    # the limiter (utils.py:249-265) is generic over the alphabet; with 20
    # Fibonacci-weighted symbols the unlimited tree is 19 deep
    counts = [1, 1]
    while len(counts) < 20:
        counts.append(counts[-1] + counts[-2])
    counter = {s: c for s, c in enumerate(counts)}
    unlimited = oc.HuffmanTable.from_frequencies(counter).get_code_table()
    assert max(b for b, _ in unlimited.values()) > 16
    _, used, table = oc.get_nbit_codec(counter, 16)
    assert max(b for b, _ in table.values()) <= 16
    assert sum(2.0 ** -b for b, _ in table.values()) == 1.0
    assert any(used[s] == 1 and counter[s] != 1 for s in counter)


# -------------------------------------------------------------------- LUTs


def _tables_for_lut_tests():
    rng = np.random.default_rng(99)
    for i in range(30):
        counter = _random_counter(rng, 0.3 + i % 4)
        yield oc.get_nbit_codec(counter, 16)[2]
    counts = [1, 1]
    while len(counts) < 16:
        counts.append(counts[-1] + counts[-2])
    yield oc.get_nbit_codec({s: c for s, c in enumerate(counts)}, 16)[2]  # 16-bit codes


@pytest.mark.parametrize("table", list(_tables_for_lut_tests()))
def test_lut_walk_decodes_every_code_under_every_padding(table):
    # brute force: each code word followed by ANY 16-bit continuation decodes
    # to its symbol and length through the two-level walk (decode.cu:86-91)
    luts = oc.get_luts_from_huffman_table(table)
    assert luts.shape[0] <= 18
    for sym, (bits, val) in table.items():
        if isinstance(sym, oc.EndOfFile):
            continue
        pad = 16 - bits
        for tail in range(1 << pad):
            w16 = (val << pad) | tail
            assert oc.lut_decode_one(luts, w16) == (sym, bits)


def test_lut_matches_worked_example_figure():
    # docs/assets/figures/lookup_table.png: codes e=0, a=10, b=110, c=1110,
    # d=1111 with 2-bit "bytes"; LUT0 maps 00->e, 10->a, 11->row 1; LUT1 maps
    # 00->b, 10->c, 11->d (the figure leaves index 01 unfilled; the builder
    # fills forward, utils.py:352-357)
    e, a, b, c, d = 0, 1, 2, 3, 4
    table = {e: (1, 0b0), a: (2, 0b10), b: (3, 0b110), c: (4, 0b1110), d: (4, 0b1111)}
    rows = oc.lut_rows(table, byte_bits=2)
    assert rows.shape == (2, 4)
    assert list(rows[0]) == [e, e, a, 4 - 1]
    assert list(rows[1]) == [b, b, c, d]


# ----------------------------------------------------------------- encoder


def _encode_by_bitstring(exps, table, eof, bpt, tpb):
    """Independent construction: the whole code string at once, gaps and
    output positions from the code start offsets."""
    codes = [format(table[s][1], f"0{table[s][0]}b") for s in exps]
    stream = "".join(codes)
    starts = np.cumsum([0] + [len(c) for c in codes[:-1]]) if codes else np.zeros(0, int)
    total = len(stream)
    if total % 8:
        eof_bits = format(table[eof][1], f"0{table[eof][0]}b")
        stream += (eof_bits + "0" * 8)[: 8 - total % 8]
    encoded = np.array([int(stream[i:i + 8], 2) for i in range(0, len(stream), 8)], np.uint8)
    chunk_bits, block_bits = 8 * bpt, 8 * bpt * tpb
    n_fb = -(-encoded.size // (bpt * tpb))
    ext_starts = list(starts) + ([total] if total % 8 else [])
    gaps = np.zeros(n_fb * tpb, np.uint8)
    seen = set()
    for s in ext_starts:
        g = s // chunk_bits
        if g not in seen:
            seen.add(g)
            gaps[g] = s % chunk_bits
    op = []
    for blk in range(n_fb):
        first = [i for i, s in enumerate(ext_starts) if s // block_bits == blk]
        op.append(first[0] if first else len(exps))
    op.append(len(exps))
    packed_gaps = np.array([(gaps[2 * i] << 4) | gaps[2 * i + 1] for i in range(gaps.size // 2)],
                           np.uint8)
    return encoded, packed_gaps, np.array(op, np.uint64)


@pytest.mark.parametrize("seed", range(25))
@pytest.mark.parametrize("geometry", [(2, 4), (4, 2), (8, 512)])
def test_encoder_matches_independent_bitstring(seed, geometry):
    bpt, tpb = geometry
    rng = np.random.default_rng(seed)
    counter = _random_counter(rng, 1.0 + seed % 3)
    syms = np.array(list(counter.keys()))
    p = np.array(list(counter.values()), float)
    n = int(rng.integers(1, 400))
    exps = rng.choice(syms, n, p=p / p.sum()).tolist()
    codec, _, table = oc.get_nbit_codec(counter, 16)
    got = oc.encode_exponents(exps, table, codec._eof, bpt, tpb)
    want = _encode_by_bitstring(exps, table, codec._eof, bpt, tpb)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_encoder_closed_form_invariants_large(oracle_native):
    rng = np.random.default_rng(3)
    flat = rng.integers(0, 256, 300_001 * 2, dtype=np.uint8)
    flat = np.where(rng.random(flat.size) < 0.7, flat & 0x9F | 0x30, flat).astype(np.uint8)
    exps, _ = oc.split_fp8(flat)
    vals, counts = np.unique(exps, return_counts=True)
    codec, _, table = oc.get_nbit_codec({int(v): int(c) for v, c in zip(vals, counts)}, 16)
    enc, gaps, op = oracle_native.encode(exps, table, codec._eof)
    lens = np.array([table[int(s)][0] for s in range(16) if int(s) in table])
    bits = np.zeros(16, np.int64)
    for s, (b, _) in table.items():
        if not isinstance(s, oc.EndOfFile):
            bits[s] = b
    starts = np.concatenate([[0], np.cumsum(bits[exps])[:-1]])
    total = int(bits[exps].sum())
    assert enc.size == -(-total // 8)
    n_fb = -(-enc.size // 4096)
    assert gaps.size == n_fb * 256 and op.size == n_fb + 1
    assert op[-1] == exps.size
    # op[b] = number of symbols starting before format-block b
    assert np.array_equal(op[:-1].astype(np.int64),
                          np.searchsorted(starts, np.arange(n_fb) * 32768, side="left"))
    # every gap nibble is the offset of the first start inside its chunk
    g_all = np.empty(gaps.size * 2, np.uint8)
    g_all[0::2], g_all[1::2] = gaps >> 4, gaps & 0xF
    chunk_first = np.searchsorted(starts, np.arange(-(-total // 64)) * 64, side="left")
    assert np.array_equal(g_all[: chunk_first.size], (starts[chunk_first] % 64).astype(np.uint8))
    assert lens.max() <= 16


# ----------------------------------------------------------- decode oracle


@pytest.mark.parametrize("seed", range(6))
def test_python_decode_round_trips(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000)) * 2
    flat = rng.integers(0, 256, n, dtype=np.uint8)
    if seed % 2:
        flat = (flat & 0x87) | 0x30  # a single exponent
    res = oc.compress_block(flat, bytes_per_thread=8, threads_per_block=512 if seed < 3 else 4)
    tpb = 512 if seed < 3 else 4
    out = oc.decode(res["luts"], res["encoded"], res["packed_other_4bits"],
                    res["output_positions"], res["gaps"], threads_per_block=tpb)
    assert np.array_equal(out, flat)


@pytest.mark.parametrize("tpb", [4, 128, 512])
def test_c_decode_equals_python_decode_and_original(tpb, oracle_native):
    rng = np.random.default_rng(tpb)
    flat = rng.normal(0, 1, 20000).astype(np.float32)
    flat = torch.from_numpy(flat).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()
    res = oc.compress_block(flat, threads_per_block=tpb)
    args = (res["luts"], res["encoded"], res["packed_other_4bits"], res["output_positions"],
            res["gaps"])
    a = oc.decode(*args, threads_per_block=tpb)
    b = oracle_native.decode(*args, threads_per_block=tpb)
    c = oracle_native.decode(*args, threads_per_block=tpb, threads=4)
    assert np.array_equal(a, flat) and np.array_equal(b, flat) and np.array_equal(c, flat)


def test_decode_clamps_to_n_elements():
    # a shorter n_elements keeps exactly the first n outputs (decode.cu:152)
    rng = np.random.default_rng(11)
    flat = rng.integers(0, 256, 5000, dtype=np.uint8)
    res = oc.compress_block(flat)
    out = oc.decode(res["luts"], res["encoded"], res["packed_other_4bits"],
                    res["output_positions"], res["gaps"], n_elements=1234)
    assert np.array_equal(out, flat[:1234])


def test_entropy_bound_on_synthetic_histogram():
    # Huffman average length lies in [H, H + 1) (Shannon), and the synthetic
    # block-quantized N(0, sigma) histogram has H of about 2.5 bits
    from ecf8_amd.synth import synthetic_fp8

    w, _ = synthetic_fp8(512, 512, 0.02, seed=0)
    exps, _ = oc.split_fp8(w.reshape(-1).view(torch.uint8).numpy())
    vals, counts = np.unique(exps, return_counts=True)
    p = counts / counts.sum()
    h = float(-(p * np.log2(p)).sum())
    table = oc.get_nbit_codec({int(v): int(c) for v, c in zip(vals, counts)}, 16)[2]
    avg = sum(table[int(v)][0] * c for v, c in zip(vals, counts)) / counts.sum()
    assert h <= avg < h + 1
    assert 2.3 < h < 2.8
    assert math.isfinite(avg)
