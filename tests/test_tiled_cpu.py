"""The tiled execution layout ECF8-T on the CPU (include/ecf8_tile.h).

* the block's Huffman code read off its LUT stack equals the code table the
  compressor built it from (every symbol's length and value);
* the C encoder's output equals an independent per-symbol Python encoding
  of the layout (stream, offsets, gaps, nibbles), byte for byte;
* every segment decodes, under the reference's own LUT rule
  (dfloat/run/decode.cu:85-91, restated by the oracle), to the Linear's FP8
  bytes in the layout's element order, and each chunk's gap is the offset
  of the first code starting in it;
* Linears the layout cannot hold are refused.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codec as oc

ROWS, GROUP, LANES, LANE_SYMS, CHUNK = 16, 128, 64, 32, 12


# a lane's symbols, in runs of 8, are its operand elements 0, 4, 1, 5, 2, 6, 3, 7
_RUN = (0, 4, 1, 5, 2, 6, 3, 7)


def _element(p, kg, i):
    lane, j = divmod(i, LANE_SYMS)
    m = 8 * (j // 8) + _RUN[j % 8]
    r, q = lane & 15, lane >> 4
    col = kg * GROUP + (16 * q + m if m < 16 else 64 + 16 * q + (m - 16))
    return p * ROWS + r, col


def _rotl32(x, n):
    return ((x << n) | (x >> (32 - n))) & 0xFFFFFFFF


def _run_dword(fp8):
    """The nibble-plane dword of one run of 8 symbols from its operand
    elements' FP8 bytes (fp8[m], m = 0..7): elements 0..3's sign and
    mantissa bits (mask 0x87 of each byte) where their bytes have them, OR
    elements 4..7's rotated left by 4 bits."""
    lo = sum((fp8[q] & 0x87) << (8 * q) for q in range(4))
    hi = sum((fp8[q + 4] & 0x87) << (8 * q) for q in range(4))
    return lo | _rotl32(hi, 4)


def _sign_mantissa(run_dword, m):
    """Bits 0x87 of operand element m's FP8 byte, read back from its run's
    dword (elements 4..7 after a 4-bit right rotation)."""
    d = run_dword if m < 4 else _rotl32(run_dword, 28)
    return (d >> (8 * (m % 4))) & 0x87


def _py_encode(w: np.ndarray, table: dict):
    """Independent restatement of the layout, symbol by symbol."""
    n, k = w.shape
    groups = k // GROUP
    stream, seg_off, gaps, other = bytearray(), [], [], bytearray()
    for p in range(n // ROWS):
        for kg in range(groups):
            seg_off.append(len(stream))
            bits, starts = "", []
            seg_other = bytearray(1024)
            run = [0] * 8
            for i in range(2048):
                r, c = _element(p, kg, i)
                b = int(w[r, c])
                e = (b >> 3) & 15
                starts.append(len(bits))
                nb, val = table[e]
                bits += format(val, f"0{nb}b")
                run[_RUN[i % 8]] = b
                if i % 8 == 7:
                    seg_other[i // 2 - 3:i // 2 + 1] = _run_dword(run).to_bytes(4, "little")
            nbytes = (len(bits) + 7) // 8
            bits += "0" * (8 * nbytes - len(bits))
            seg = bytes(int(bits[8 * t:8 * t + 8], 2) for t in range(nbytes))
            seg += b"\0" * ((-len(seg)) % 4)
            stream += seg
            g = [0] * 64
            for c in range(64):
                first = next((s for s in starts if s >= CHUNK * 8 * c), None)
                if first is not None and first - CHUNK * 8 * c < CHUNK * 8:
                    g[c] = first - CHUNK * 8 * c
            gaps += [sum(g[8 * wd + t] << (4 * t) for t in range(8)) for wd in range(8)]
            other += seg_other
    seg_off.append(len(stream))
    stream += b"\0" * 16
    return (np.frombuffer(bytes(stream), np.uint8), np.array(seg_off, np.uint32),
            np.array(gaps, np.uint32), np.frombuffer(bytes(other), np.uint8))


def _weights(n, k, seed):
    from ecf8_amd.synth import synthetic_fp8

    w, _ = synthetic_fp8(-(-n // 128) * 128, k, 0.02, seed=seed)  # 128x128 scale blocks
    return w[:n].contiguous()


def _compressed(w):
    from dfloat.compress import compress_flat

    return compress_flat(w.reshape(-1))


def test_code_read_off_the_luts_is_the_compressors_code():
    from ecf8_amd.tiled import code_from_luts

    for seed, (n, k) in enumerate([(128, 256), (256, 512), (128, 1024)]):
        res = _compressed(_weights(n, k, seed))
        bits, vals = code_from_luts(res["luts"])
        for sym, (nb, val) in res["table"].items():
            if isinstance(sym, (int, np.integer)):
                assert (bits[sym], vals[sym]) == (nb, val), sym
        present = {int(s) for s in res["table"] if isinstance(s, (int, np.integer))}
        assert {s for s in range(16) if bits[s]} == present


def test_code_read_off_the_luts_of_skewed_and_long_codes():
    """1-bit codes (a dominant exponent) and 16-bit codes (Fibonacci counts,
    two LUT levels) are recovered too."""
    from ecf8_amd.tiled import code_from_luts

    counts = [1, 1]
    while len(counts) < 16:
        counts.append(counts[-1] + counts[-2])
    for counter in ({s: c for s, c in enumerate(counts)}, {12: 900, 11: 50, 13: 40, 3: 10}):
        _, _, table = oc.get_nbit_codec(counter, 16)
        luts = oc.get_luts_from_huffman_table(table)
        bits, vals = code_from_luts(luts)
        for sym, (nb, val) in table.items():
            if isinstance(sym, int):
                assert (bits[sym], vals[sym]) == (nb, val), sym


@pytest.mark.parametrize("n,k,seed", [(16, 128, 1), (32, 256, 2), (48, 384, 3)])
def test_encoder_equals_a_python_restatement(n, k, seed):
    from ecf8_amd.tiled import code_from_luts, tile_encode

    w = _weights(n, k, seed)
    res = _compressed(w)
    bits, vals = code_from_luts(res["luts"])
    enc = tile_encode(w, bits, vals, n_threads=3)
    table = {s: (int(bits[s]), int(vals[s])) for s in range(16) if bits[s]}
    stream, seg_off, gaps, other = _py_encode(w.view(torch.uint8).numpy(), table)
    assert np.array_equal(enc["seg_off"].numpy().view(np.uint32), seg_off)
    assert np.array_equal(enc["stream"].numpy(), stream)
    assert np.array_equal(enc["gaps"].numpy().view(np.uint32), gaps)
    assert np.array_equal(enc["other"].numpy(), other)


def test_segments_decode_under_the_reference_rule():
    _check_segments(_weights(64, 512, 7), _compressed)


def _check_segments(w, compressed):
    from ecf8_amd.tiled import code_from_luts, tile_encode

    n, k = w.shape
    wb = w.view(torch.uint8).numpy()
    res = compressed(w)
    luts = res["luts"].numpy()
    bits, vals = code_from_luts(luts)
    enc = tile_encode(w, bits, vals)
    stream = enc["stream"].numpy()
    seg_off = enc["seg_off"].numpy().view(np.uint32)
    gaps = enc["gaps"].numpy().view(np.uint32)
    other = enc["other"].numpy()
    groups = k // GROUP
    assert seg_off.size == (n // ROWS) * groups + 1
    assert stream.size == seg_off[-1] + 16 and (seg_off % 4 == 0).all()
    for s in range(seg_off.size - 1):
        p, kg = divmod(s, groups)
        base = int(seg_off[s])
        n_chunks = -(-(int(seg_off[s + 1]) - base) // CHUNK)
        assert n_chunks <= 64
        pos, starts = 0, []
        for i in range(2048):
            w16 = 0
            for t in range(3):  # 24 bits from the current position
                j = base + (pos >> 3) + t
                w16 = (w16 << 8) | int(stream[j])
            w16 = (w16 >> (8 - (pos & 7))) & 0xFFFF
            sym, ln = oc.lut_decode_one(luts, w16)
            starts.append(pos)
            at = s * 1024 + (i // 8) * 4
            d = int.from_bytes(other[at:at + 4].tobytes(), "little")
            r, c = _element(p, kg, i)
            assert (_sign_mantissa(d, _RUN[i % 8]) | sym << 3) == wb[r, c], (s, i)
            pos += ln
        for c in range(n_chunks):
            g = (int(gaps[s * 8 + c // 8]) >> (4 * (c % 8))) & 15
            first = next(x for x in starts + [10 ** 9] if x >= 96 * c)
            if first < 96 * c + 96:
                assert first == 96 * c + g, (s, c)


def test_code_recovery_from_an_incomplete_code():
    """A Qwen3-MoE-shaped expert block (intermediate 256) whose Huffman code
    leaves 4 of the 65536 16-bit windows without a code (Kraft sum
    1 - 2^-14): the LUT builder fills them with exponent 0, ahead of
    exponent 0's real 13-bit code.  Every recovered code has the
    compressor's length and decodes to its symbol under the reference rule,
    and a Linear of the block encodes and decodes segment by segment."""
    from dfloat.compress import compress_flat
    from ecf8_amd.synth import flat_block, synthetic_block
    from ecf8_amd.tiled import code_from_luts

    shapes = {"gate_proj": (256, 2048, 0.02), "up_proj": (256, 2048, 0.02),
              "down_proj": (2048, 256, 0.02)}
    weights = synthetic_block(shapes, seed=400016)
    flat, _ = flat_block(weights)
    res = compress_flat(flat)
    table = {s: v for s, v in res["table"].items() if isinstance(s, (int, np.integer))}
    assert sum(2.0 ** -nb for nb, _ in table.values()) < 1.0  # incomplete
    luts = res["luts"].numpy()
    bits, vals = code_from_luts(luts)
    for sym, (nb, _) in table.items():
        assert bits[sym] == nb, sym
        lo = int(vals[sym]) << (16 - nb)
        for wnd in range(lo, lo + (1 << (16 - nb))):
            assert oc.lut_decode_one(luts, wnd) == (sym, nb), (sym, wnd)
    # the compressor's code of exponent 0 differs from the first window
    # decoding to 0: the case a first-window rule gets wrong
    nb0, val0 = table[0]
    first0 = next(wnd for wnd in range(65536) if oc.lut_decode_one(luts, wnd)[0] == 0)
    assert first0 >> (16 - nb0) != val0
    _check_segments(weights["gate_proj"][0][:32].contiguous(), lambda _w: res)


def test_layout_refusals():
    from ecf8_amd.tiled import code_from_luts, tile_encode
    from ecf8_amd._lib import ECF8Error

    w = _weights(32, 256, 4)
    res = _compressed(w)
    bits, vals = code_from_luts(res["luts"])
    with pytest.raises(ECF8Error, match="geometry|unsupported"):
        tile_encode(w[:24], bits, vals)       # rows not a multiple of 16
    missing = bits.copy()
    missing[int(np.argmax(bits))] = 0          # an exponent present without a code
    with pytest.raises(ECF8Error):
        tile_encode(w, missing, vals)
    # 4 bits per exponent (16 equally likely exponents): 1024-byte segments
    rng = np.random.default_rng(0)
    e = rng.integers(0, 16, (32, 256)).astype(np.uint8)
    flat = torch.from_numpy((e << 3).astype(np.uint8))
    uni_bits, uni_vals = np.full(16, 4, np.uint8), np.arange(16, dtype=np.uint32)
    with pytest.raises(ECF8Error, match="too small"):
        tile_encode(flat, uni_bits, uni_vals)


def test_code_read_off_luts_whose_eof_code_is_the_lowest_key():
    """A code whose EOF code is all zeros leaves the lowest LUT entries to
    the builder's default symbol 0, here absent from the data (length 0):
    those windows carry no symbol, and every present symbol's code is still
    recovered."""
    from ecf8_amd.tiled import code_from_luts

    _, _, table = oc.get_nbit_codec({11: 900, 12: 150}, 16)
    luts = oc.get_luts_from_huffman_table(table)
    assert luts[-1][0] == 0 and oc.lut_decode_one(luts, 0)[0] == 0  # code-less windows
    bits, vals = code_from_luts(luts)
    for sym, (nb, val) in table.items():
        if isinstance(sym, int):
            assert (bits[sym], vals[sym]) == (nb, val), sym
    assert {s for s in range(16) if bits[s]} == {11, 12}
