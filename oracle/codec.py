"""Pure-Python restatement of the reference ECF8 codec (test infrastructure).

Every function cites the reference file:line it follows.  These are written
for clarity, not speed: the per-symbol loops are only used on small inputs;
``oracle/ecf8_oracle.c`` restates the same encoder and decode rule for large
inputs.
"""

from __future__ import annotations

import heapq
from copy import copy

import numpy as np

# --------------------------------------------------------------------------
# FP8 e4m3fn split / merge                       dfloat/utils.py:207-227
# --------------------------------------------------------------------------


def split_fp8(w_u8: np.ndarray):
    """Return (exponents u8[n], packed_other_4bits u8[n/2]).

    Follows dfloat/utils.py:212-225: exponent = (b >> 3) & 0xF,
    other = ((b >> 4) & 0x8) | (b & 0x7), and pairs are packed with the even
    element in the high nibble.
    """
    w = np.asarray(w_u8, dtype=np.uint8).reshape(-1)
    assert w.size % 2 == 0, "reference requires an even element count (utils.py:224)"
    exps = (w >> 3) & 0xF
    other = ((w >> 4) & 0x8) | (w & 0x7)
    pairs = other.reshape(-1, 2)
    packed = ((pairs[:, 0] << 4) | pairs[:, 1]).astype(np.uint8)
    return exps.astype(np.uint8), packed


def merge_fp8(exps: np.ndarray, packed: np.ndarray) -> np.ndarray:
    """Inverse of split_fp8: the byte the decoder writes (decode.cu:174-175).

    out = (o & 8) << 4 | e << 3 | (o & 7), with o taken from the high nibble
    for even indices and the low nibble for odd ones.
    """
    exps = np.asarray(exps, dtype=np.uint8)
    packed = np.asarray(packed, dtype=np.uint8)
    other = np.empty(packed.size * 2, dtype=np.uint8)
    other[0::2] = packed >> 4
    other[1::2] = packed & 0xF
    return (((other & 0x8) << 4) | (exps << 3) | (other & 0x7)).astype(np.uint8)


# --------------------------------------------------------------------------
# Huffman code table: restatement of dahuffman's HuffmanCodec.from_frequencies
# (third-party dependency used at dfloat/utils.py:7,240,259; unpinned in
# requirements.txt:34; published algorithm of dahuffman 0.4.x).
#
# A heap of (frequency, [(symbol, (bitsize, value)), ...]) entries, one per
# symbol plus an end-of-file pseudo-symbol of frequency 1.  The two smallest
# entries a, b are popped and merged; every code in a gets a new leading 0,
# every code in b a new leading 1 (value += 1 << bitsize).  Ties in frequency
# are broken by Python's list comparison, i.e. by the first symbol of each
# entry, with the EOF symbol ordering before every other symbol.
# --------------------------------------------------------------------------


class EndOfFile:
    """EOF pseudo-symbol; compares smaller than every other symbol."""

    def __repr__(self):
        return "_EOF"

    def __lt__(self, other):
        return True

    def __gt__(self, other):
        return False

    def __eq__(self, other):
        return other.__class__ == self.__class__

    def __hash__(self):
        return hash(self.__class__)


EOF = EndOfFile()


class HuffmanTable:
    """Minimal stand-in for the dahuffman codec object the reference reads.

    The reference only touches ``codec._table`` (utils.py:408),
    ``codec._eof`` (utils.py:447) and ``codec.get_code_table()``
    (utils.py:241,260).
    """

    def __init__(self, table: dict, eof=EOF):
        self._table = table
        self._eof = eof

    def get_code_table(self):
        return self._table

    @classmethod
    def from_frequencies(cls, frequencies: dict, eof=EOF):
        heap = [(f, [(s, (0, 0))]) for s, f in frequencies.items()]
        if eof not in frequencies:
            heap.append((1, [(eof, (0, 0))]))
        heapq.heapify(heap)
        while len(heap) > 1:
            a = heapq.heappop(heap)
            b = heapq.heappop(heap)
            merged = (
                a[0] + b[0],
                [(s, (n + 1, v)) for (s, (n, v)) in a[1]]
                + [(s, (n + 1, (1 << n) + v)) for (s, (n, v)) in b[1]],
            )
            heapq.heappush(heap, merged)
        return cls(dict(heap[0][1]), eof=eof)


def get_nbit_codec(counter: dict, max_n_bits: int = 16):
    """Length-limited code table, dfloat/utils.py:239-267.

    While the longest code exceeds ``max_n_bits``, the ``min_k`` rarest
    symbols (numpy argpartition over the counts in counter order) get count 1
    and the table is rebuilt, with ``min_k`` growing by one per round.
    """
    codec = HuffmanTable.from_frequencies(counter)
    table = codec.get_code_table()
    max_len = max(length for length, _ in table.values())
    compressed_codec, compressed_counter = codec, counter
    min_k = 2
    freq = np.array(list(counter.values()))
    while max_len > max_n_bits:
        min_indices = np.argpartition(freq, min_k)[:min_k]
        min_k += 1
        min_keys = np.array(list(counter.keys()))[min_indices]
        compressed_counter = copy(counter)
        for k in min_keys:
            compressed_counter[k] = 1
        compressed_codec = HuffmanTable.from_frequencies(compressed_counter)
        table = compressed_codec.get_code_table()
        max_len = max(length for length, _ in table.values())
    return compressed_codec, compressed_counter, table


# --------------------------------------------------------------------------
# Hierarchical decode LUTs                        dfloat/utils.py:270-370
# --------------------------------------------------------------------------


def lut_rows(table: dict, byte_bits: int = 8) -> np.ndarray:
    """The decode rows of get_luts_from_huffman_table (utils.py:271-357) for
    a ``byte_bits``-wide index: row 0 for codes whose (len-1)//byte_bits ==
    0, one extra row per distinct first byte of a longer code (rows ordered by
    first appearance, stable-sorted by prefix length, :271-289); each row
    filled forward from left-justified keys (:352-357); pointers are
    2**byte_bits - row (:339).  byte_bits is 8 in the reference; 2 gives the
    worked example of docs/assets/figures/lookup_table.png."""
    B = byte_bits
    W = 1 << B

    def code_str(bits, val):
        return bin(val)[2:].rjust(bits, "0")

    prefixes = [""]
    for symbol, (bits, val) in table.items():
        if not isinstance(symbol, (int, np.integer)):
            continue
        prefix_len = (bits - 1) - (bits - 1) % B
        prefix = code_str(bits, val)[:prefix_len]
        if prefix not in prefixes:
            prefixes.append(prefix)
    prefixes.sort(key=len)

    luts = np.zeros((len(prefixes), W), dtype=np.uint8)
    for prefix_idx, prefix in enumerate(prefixes):
        entries = {}
        prefix_n_bytes = len(prefix) // B
        prefix_n_bits = prefix_n_bytes * B
        for symbol, (bits, val) in table.items():
            if not isinstance(symbol, (int, np.integer)):
                continue
            s = code_str(bits, val)
            if not s.startswith(prefix):
                continue
            if (bits - 1) // B == prefix_n_bytes:
                key = int(s[prefix_n_bits:].ljust(B, "0"), 2)
                value = int(symbol)
            else:
                assert (bits - 1) // B > prefix_n_bytes
                key = int(s[prefix_n_bits : prefix_n_bits + B], 2)
                value = W - prefixes.index(s[: prefix_n_bits + B])
            if key in entries and entries[key] != value:
                raise ValueError(f"Key {key} already exists in {entries}")
            entries[key] = value
        cur = 0
        for k in range(W):
            if k in entries:
                cur = entries[k]
            luts[prefix_idx, k] = cur
    return luts


def get_luts_from_huffman_table(table: dict) -> np.ndarray:
    """u8[n_luts, 256]: the decode rows of lut_rows(table, 8) followed by the
    code length of each symbol (utils.py:359-369)."""
    rows = lut_rows(table, 8)
    lens = np.zeros((1, 256), dtype=np.uint8)
    for symbol, (bits, val) in table.items():
        if isinstance(symbol, (int, np.integer)):
            lens[0, int(symbol)] = bits
    return np.concatenate((rows, lens), axis=0)


# --------------------------------------------------------------------------
# Bitstream encoder                               dfloat/utils.py:373-499
# --------------------------------------------------------------------------


def encode_exponents(exponents, table: dict, eof=EOF, bytes_per_thread: int = 8,
                     threads_per_block: int = 512):
    """Per-symbol restatement of _encode_exponents_for_cuda (utils.py:373-499).

    Returns (encoded u8[n_bytes], packed gaps u8, output_positions u64[nb+1]).
    """
    bits_per_thread = 8 * bytes_per_thread
    bits_per_block = bits_per_thread * threads_per_block
    encoded, gaps, output_positions = [], [], []
    buffer = size = total_size = element_count = 0
    for symbol in exponents:
        if total_size // bits_per_thread + 1 > len(gaps):          # :392
            gaps.append(total_size % bits_per_thread)
        if total_size // bits_per_block + 1 > len(output_positions):  # :405
            output_positions.append(element_count)
        bits, val = table[symbol]
        buffer = (buffer << bits) + val
        size += bits
        total_size += bits
        element_count += 1
        while size >= 8:                                             # :422
            byte = buffer >> (size - 8)
            encoded.append(byte)
            buffer -= byte << (size - 8)
            size -= 8
    if size > 0:                                                     # :439
        if total_size // (8 * bytes_per_thread) + 1 > len(gaps):
            gaps.append(total_size % bits_per_thread)
        if total_size // bits_per_block + 1 > len(output_positions):
            output_positions.append(element_count)
        bit, val = table[eof]
        buffer = (buffer << bit) + val
        size += bit
        byte = buffer >> (size - 8) if size >= 8 else buffer << (8 - size)
        encoded.append(byte)
    output_positions.append(len(exponents))                          # :463
    n_bytes = len(encoded)
    blocks = -(-n_bytes // (threads_per_block * bytes_per_thread))   # :471
    gaps.extend([0] * (blocks * threads_per_block - len(gaps)))       # :476
    bits = [int(c) for g in gaps for c in format(g, "04b")]          # :482
    return (
        np.frombuffer(bytes(encoded), dtype=np.uint8).copy(),
        np.packbits(np.array(bits, dtype=np.uint8)) if bits else np.zeros(0, np.uint8),
        np.array(output_positions, dtype=np.uint64),
    )


# --------------------------------------------------------------------------
# Decode rule                                     dfloat/run/decode.cu:15-211
# --------------------------------------------------------------------------


def lut_decode_one(luts: np.ndarray, window16: int):
    """One symbol from the next 16 bits (decode.cu:86-91): returns (sym, len)."""
    n_luts = luts.shape[0]
    v = int(luts[0, window16 >> 8])
    if v >= 240:
        v = int(luts[256 - v, window16 & 0xFF])
    return v, int(luts[n_luts - 1, v])


def decode_chunk_symbols(luts, encoded, gaps_packed, g, bytes_per_thread=8):
    """Symbols owned by chunk g: those starting at bit offsets c with
    gap_g <= c < 8*bytes_per_thread, read from the chunk plus a 2-byte
    look-ahead (decode.cu:42-112, 156-204).  Bytes past the stream read as 0
    (the reference reads uninitialised registers there; only symbols past
    the last output position can depend on them)."""
    n_bytes = encoded.size
    nb = bytes_per_thread + 2
    window = 0
    for i in range(nb):
        j = g * bytes_per_thread + i
        window = (window << 8) | (int(encoded[j]) if j < n_bytes else 0)
    total_bits = 8 * nb
    gb = int(gaps_packed[g // 2])
    gap = (gb >> 4) & 0xF if g % 2 == 0 else gb & 0xF
    pos, syms = gap, []
    while pos < 8 * bytes_per_thread:
        w16 = (window >> (total_bits - pos - 16)) & 0xFFFF
        v, ln = lut_decode_one(luts, w16)
        if ln == 0:
            # only the EOF pad bits reach a code-less entry (the LUT fill
            # starts from symbol 0, utils.py:352); the reference would spin
            # here, and every later symbol lies past the last output anyway
            break
        syms.append(v)
        pos += ln
    return syms


def decode(luts, encoded, packed_other_4bits, output_positions, gaps,
           n_elements=None, threads_per_block=512, bytes_per_thread=8):
    """Full decode of one compressed block: returns u8[n_elements] FP8 bytes.

    Format-block b covers chunks [b*tpb, (b+1)*tpb); its symbols, in chunk
    order, land at output_positions[b] + k, clamped to the block's range and
    to n_elements (decode.cu:114-152, 207-210).
    """
    luts = np.asarray(luts, dtype=np.uint8)
    encoded = np.asarray(encoded, dtype=np.uint8)
    packed = np.asarray(packed_other_4bits, dtype=np.uint8)
    op = np.asarray(output_positions).view(np.uint64).astype(np.int64)
    gaps = np.asarray(gaps, dtype=np.uint8)
    n = packed.size * 2 if n_elements is None else int(n_elements)
    n_bytes = encoded.size
    blocks = -(-n_bytes // (threads_per_block * bytes_per_thread))
    exps = np.zeros(n, dtype=np.uint8)
    for b in range(blocks):
        start, end = int(op[b]), min(int(op[b + 1]), n)
        syms = []
        for t in range(threads_per_block):
            syms.extend(decode_chunk_symbols(luts, encoded, gaps,
                                             b * threads_per_block + t,
                                             bytes_per_thread))
            if len(syms) >= end - start:
                break
        take = max(0, end - start)
        exps[start:start + take] = syms[:take]
    return merge_fp8(exps, packed[: n // 2])


# --------------------------------------------------------------------------
# Whole-block pipeline (scripts/compress.py:197-247 without file I/O)
# --------------------------------------------------------------------------


def compress_block(flat_u8: np.ndarray, bytes_per_thread=8, threads_per_block=512):
    """Counter in ascending symbol order (compress.py:205,213-215) -> table ->
    LUTs -> encoder.  Returns a dict with the reference's on-disk names."""
    exps, packed = split_fp8(flat_u8)
    vals, counts = np.unique(exps, return_counts=True)
    counter = {int(v): int(c) for v, c in zip(vals, counts)}
    codec, _, table = get_nbit_codec(counter, 16)
    luts = get_luts_from_huffman_table(table)
    encoded, gaps, op = encode_exponents(exps.tolist(), codec._table, codec._eof,
                                         bytes_per_thread, threads_per_block)
    return {
        "luts": luts,
        "encoded": encoded,
        "packed_other_4bits": packed,
        "output_positions": op,
        "gaps": gaps,
        "table": table,
    }
