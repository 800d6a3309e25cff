"""Huffman code tables with the code assignment the reference's compressor
produces.

The reference builds its codebook with the third-party ``dahuffman`` package
(``HuffmanCodec.from_frequencies``, called at dfloat/utils.py:240 and :259)
and reads back only ``codec._table`` (symbol -> (bit length, code value)),
``codec._eof`` and ``codec.get_code_table()``.  Decoding does not depend on
which optimal code is chosen (the LUTs carry it), but writing checkpoints a
reference decoder reads byte-identically does, so this module reproduces
dahuffman's merge order:

* leaves are the symbols plus an end-of-file pseudo-symbol of weight 1;
* the two lightest subtrees are merged, lighter first; equal weights are
  ordered by the first symbol of each subtree (EOF before every symbol);
* the first-popped subtree becomes the 0 branch, the second the 1 branch,
  and the table lists symbols left to right.
"""

from __future__ import annotations

import heapq
from copy import copy

import numpy as np


class EndOfFile:
    """End-of-file pseudo-symbol (orders before every real symbol)."""

    _instance = None

    def __new__(cls):
        if cls._instance is None:
            cls._instance = super().__new__(cls)
        return cls._instance

    def __repr__(self):
        return "_EOF"

    def __lt__(self, other):
        return True

    def __gt__(self, other):
        return False

    def __eq__(self, other):
        return isinstance(other, EndOfFile)

    def __hash__(self):
        return hash(EndOfFile)


_EOF = EndOfFile()


def _order_key(symbol):
    return (0, 0) if isinstance(symbol, EndOfFile) else (1, symbol)


class HuffmanCodec:
    """Code table holder with the attributes the reference's encoder reads."""

    def __init__(self, table: dict, eof=_EOF):
        self._table = table
        self._eof = eof

    def get_code_table(self) -> dict:
        return self._table

    @classmethod
    def from_frequencies(cls, frequencies: dict, eof=_EOF) -> "HuffmanCodec":
        leaves = list(frequencies.items())
        if eof not in frequencies:
            leaves.append((eof, 1))
        # node = symbol (leaf) or (left, right); heap rows are
        # (weight, order key of the subtree's first symbol, node id)
        nodes = [sym for sym, _ in leaves]
        heap = [(w, _order_key(sym), i) for i, (sym, w) in enumerate(leaves)]
        heapq.heapify(heap)
        children = {}
        while len(heap) > 1:
            wa, ka, a = heapq.heappop(heap)
            wb, _, b = heapq.heappop(heap)
            nid = len(nodes)
            nodes.append(None)
            children[nid] = (a, b)
            heapq.heappush(heap, (wa + wb, ka, nid))
        table = {}
        root = heap[0][2]
        stack = [(root, 0, 0)]
        while stack:  # depth-first, 0-branch first: the reference's listing order
            nid, depth, value = stack.pop()
            if nid in children:
                a, b = children[nid]
                stack.append((b, depth + 1, (value << 1) | 1))
                stack.append((a, depth + 1, value << 1))
            else:
                table[nodes[nid]] = (depth, value)
        return cls(table, eof)


def get_nbit_codec(counter: dict, max_n_bits: int = 16):
    """Length-limited codebook (dfloat/utils.py:239-267): while the longest
    code exceeds ``max_n_bits`` the ``k`` rarest symbols (numpy argpartition
    over the counts, k = 2, 3, ...) are given count 1 and the table rebuilt.
    For 4-bit exponents the loop never runs: 16 symbols plus EOF are 17
    leaves, whose deepest possible code is 16 bits.  Returns (codec, counter
    used, code table)."""
    codec = HuffmanCodec.from_frequencies(counter)
    table = codec.get_code_table()
    longest = max(bits for bits, _ in table.values())
    used = counter
    k = 2
    freq = np.array(list(counter.values()))
    keys = np.array(list(counter.keys()))
    while longest > max_n_bits:
        rare = keys[np.argpartition(freq, k)[:k]]
        k += 1
        used = copy(counter)
        for sym in rare:
            used[sym] = 1
        codec = HuffmanCodec.from_frequencies(used)
        table = codec.get_code_table()
        longest = max(bits for bits, _ in table.values())
    return codec, used, table
