// Construction of the derived decode tables (layout in ecf8_layout.h) from a
// compressed block's LUT stack, written once for both builders: the host
// builder (ecf8_tables.cpp) runs every step in a loop, the device builder
// (build_table_kernel in ecf8_table_kernel.hip) runs each step's independent
// items across a workgroup.  Both therefore produce the same bytes.
//
// The tables reproduce the reference decode rule (dfloat/run/decode.cu:85-91)
//   v = L0[W >> 8];  if (v >= 240) v = L[256 - v][W & 0xFF];  len = Llen[v]
// on the 16-bit window W at a code start.
//
// Central quantity: det(m, q), the rule's result shared by every 16-bit
// window that starts with the m-bit prefix q, packed as (symbol << 8) | len,
// or kDetMixed when windows with that prefix disagree, or kDetInvalid when
// the rule leaves the LUT stack or yields a value above 15.  It is read off
// "range trees": for the first-level row (tree 0) and each second-level row
// r (tree r), a heap over the row's 256 entries where a node holds the
// common result of its range, or kDetMixed.
#ifndef ECF8_TABLE_BUILD_H
#define ECF8_TABLE_BUILD_H

#include <stdint.h>

#include "ecf8.h"
#include "ecf8_layout.h"

namespace ecf8 {

constexpr int16_t kDetInvalid = -1;
constexpr int16_t kDetMixed = -2;
constexpr int kTreeNodes = 512;                    // heap: root 1, leaves 256..511
constexpr int kMaxTrees = ECF8_MAX_LUTS - 1;       // first level + 16 second-level rows
constexpr int kTableWords = ECF8_TABLE_BYTES / 4;  // automaton entries + kind word
constexpr int kKindWord = kDfaEntries;             // word holding the table kind
// canonical prefix index: key (1 << m) | q for m = 1..15 maps to key - 2
constexpr int kPrefixKeys = (1 << 16) - 2;

struct TableScratch {
  uint8_t luts[ECF8_MAX_LUTS * 256];
  int16_t tree[kMaxTrees][kTreeNodes];
  uint32_t pending[kDfaMaxPending];  // keys of the automaton's pending rows
  int n_luts;
  int n_pending;
};

ECF8_HD inline int16_t rule_value(const TableScratch &s, int v) {
  return v > 15 ? kDetInvalid : (int16_t)((v << 8) | s.luts[(s.n_luts - 1) * 256 + v]);
}

// Rows that hold second-level entries: 1 .. n_luts - 2.
ECF8_HD inline int second_level_rows(const TableScratch &s) { return s.n_luts - 2; }

// Leaf i of tree t.  Tree 0's leaves need the roots of the second-level
// trees, so those are finished first.
ECF8_HD inline int16_t tree_leaf(const TableScratch &s, int t, int i) {
  if (t > 0) return rule_value(s, s.luts[t * 256 + i]);
  const int v = s.luts[i];
  if (v < 240) return rule_value(s, v);
  const int row = 256 - v;
  if (row > second_level_rows(s)) return kDetInvalid;
  return s.tree[row][1];
}

ECF8_HD inline int16_t tree_combine(int16_t a, int16_t b) { return a == b ? a : kDetMixed; }

// The rule on one 16-bit window.
ECF8_HD inline int16_t rule16(const TableScratch &s, uint32_t w) {
  int v = s.luts[w >> 8];
  if (v >= 240) {
    const int row = 256 - v;
    if (row > second_level_rows(s)) return kDetInvalid;
    v = s.luts[row * 256 + (w & 0xFF)];
  }
  return rule_value(s, v);
}

// det(m, q) for 0 <= m <= 16 once the trees are complete.
ECF8_HD inline int16_t det(const TableScratch &s, int m, uint32_t q) {
  if (m >= 16) return rule16(s, q & 0xFFFFu);
  if (m < 8) return s.tree[0][(1u << m) | q];
  const int j = m - 8;
  const int v = s.luts[q >> j];
  if (v < 240) return rule_value(s, v);
  const int row = 256 - v;
  if (row > second_level_rows(s)) return kDetInvalid;
  return s.tree[row][(1u << j) | (q & ((1u << j) - 1))];
}

// A prefix the automaton must hold as a state: the bits read since the
// code start do not fix the symbol yet, or fix one whose code is longer.
ECF8_HD inline bool prefix_pending(const TableScratch &s, uint32_t key) {
  const int m = 31 - __builtin_clz(key);
  const int16_t d = det(s, m, key & ((1u << m) - 1));
  return d == kDetMixed || (d >= 0 && (d & 0xFF) > m);
}

// Canonical prefix index <-> key.
ECF8_HD inline uint32_t prefix_key(int index) { return (uint32_t)index + 2; }

// Row of a pending prefix; -1 if it is not one (cannot happen for prefixes
// the walk meets, since every pending prefix of 1..15 bits has a row).
ECF8_HD inline int pending_row(const TableScratch &s, uint32_t key) {
  for (int i = 0; i < s.n_pending; ++i)
    if (s.pending[i] == key) return kDfaFirstPendingRow + i;
  return -1;
}

// One automaton entry: decode `nbits` input bits `in` after the pending
// prefix `pk` ((1 << length) | bits; 1 = at a code start).  A symbol is
// emitted as soon as the bits read fix it.  A symbol whose rule result is
// fixed only by bits past its own length (the LUT range of the EOF code,
// filled with the preceding symbol) "rewinds": decoding resumes inside the
// bits already read.  Returns false when the LUTs do not fit the automaton
// (a length the format cannot hold, a rule result outside the stack, or
// more than 4 symbols in one byte without a rewind, i.e. a 1-bit code).
ECF8_HD inline bool dfa_entry(const TableScratch &s, uint32_t pk, uint32_t in, int nbits,
                              uint32_t *entry) {
  const int m = 31 - __builtin_clz(pk);
  const uint64_t t = ((uint64_t)(pk & ((1u << m) - 1)) << nbits) | in;
  const int len = m + nbits;
  int pos = 0, count = 0, next = -1;
  bool rewound = false;
  uint32_t syms = 0;
  for (;;) {
    const int avail = len - pos;
    if (avail == 0) {
      next = 0;
      break;
    }
    const int k = avail < 16 ? avail : 16;
    const uint32_t q = (uint32_t)(t >> (avail - k)) & ((1u << k) - 1);
    const int r = det(s, k, q);
    if (r >= 0 && (r & 0xFF) > 16) return false;
    if (r == kDetMixed || (r >= 0 && (r & 0xFF) > avail)) {
      // avail < 16 here: a 16-bit window always fixes the rule's result
      next = pending_row(s, (1u << avail) | (uint32_t)(t & ((1u << avail) - 1)));
      if (next < 0) return false;
      break;
    }
    if (r < 0) return false;
    const int l = r & 0xFF;
    if (l == 0) {  // code-less entry: the reference's decode of the chunk stops
      next = kDfaExactRow;
      break;
    }
    if (det(s, l, q >> (k - l)) != r) rewound = true;
    if (count == kDfaMaxSyms) {
      if (!rewound) return false;
      next = kDfaExactRow;
      break;
    }
    syms |= (uint32_t)(r >> 8) << (4 * count);
    ++count;
    pos += l;
  }
  *entry = (uint32_t)(4 * count) | ((uint32_t)next << 10) | (syms << 16);
  return true;
}

// Automaton entry e (0 .. kDfaEntries-1), pending rows known.
ECF8_HD inline bool dfa_table_entry(const TableScratch &s, int e, uint32_t *out) {
  const uint32_t exact = (uint32_t)kDfaExactRow << 10;
  if (e >= kDfaSkipByte) {
    *out = (uint32_t)(e - kDfaSkipByte) << 10;
    return true;
  }
  const int row = e >> 8, b = e & 0xFF;
  if (row == 0) return dfa_entry(s, 1u, (uint32_t)b, 8, out);
  if (row < kDfaExactRow) return dfa_entry(s, 1u, (uint32_t)b & ((1u << (8 - row)) - 1), 8 - row, out);
  const int p = row - kDfaFirstPendingRow;
  if (row == kDfaExactRow || p >= s.n_pending) {
    *out = exact;  // rows past the pending ones are never reached
    return true;
  }
  return dfa_entry(s, s.pending[p], (uint32_t)b, 8, out);
}

// Multi-symbol entry for the 12-bit window w.  A symbol is accepted only
// while the rule's result provably does not depend on the bits after the
// window (every LUT entry the unknown bits could select holds the same
// value), so the table is exact for any LUT stack.
ECF8_HD inline uint32_t multi_entry(const TableScratch &s, int w) {
  const uint8_t *len_row = s.luts + 256 * (s.n_luts - 1);
  uint32_t syms = 0, mask = 0;
  int n = 0, off = 0;
  while (n < kMaxSymsPerEntry && off < kWinBits) {
    const int known = kWinBits - off;  // window bits from this symbol's start
    const int kb = known < 8 ? known : 8;
    const int idx = ((w >> (known - kb)) & ((1 << kb) - 1)) << (8 - kb);
    const int span = 1 << (8 - kb);
    int v = s.luts[idx];
    bool fixed = true;
    for (int x = 1; x < span; ++x) fixed &= s.luts[idx + x] == v;
    if (!fixed) break;
    if (v >= 240) {
      const int row = 256 - v;
      if (row > second_level_rows(s)) break;
      const int known2 = known - 8;  // bits of the second byte inside the window
      const int kb2 = known2 <= 0 ? 0 : (known2 < 8 ? known2 : 8);
      const int idx2 = kb2 ? ((w >> (known2 - kb2)) & ((1 << kb2) - 1)) << (8 - kb2) : 0;
      const int span2 = 1 << (8 - kb2);
      const uint8_t *r = s.luts + 256 * row;
      v = r[idx2];
      for (int x = 1; x < span2; ++x) fixed &= r[idx2 + x] == v;
      if (!fixed) break;
    }
    const int len = len_row[v];
    if (len == 0 || len > known || v > 15) break;
    syms |= (uint32_t)v << (4 * n);
    mask |= 1u << off;
    ++n;
    off += len;
  }
  return n ? (syms | (mask << 16) | ((uint32_t)off << 28)) : 0u;
}

}  // namespace ecf8

#endif  // ECF8_TABLE_BUILD_H
