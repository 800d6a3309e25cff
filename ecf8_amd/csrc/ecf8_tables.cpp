// Host construction of the derived decode tables (layout in ecf8_layout.h)
// from a compressed block's LUT stack.  Both tables reproduce the reference
// decode rule (dfloat/run/decode.cu:85-91) exactly; they are built once per
// compressed block, at load time, like the reference's shared_mem_size
// (dfloat/run/run.py:453-458).

#include <stdint.h>
#include <string.h>

#include <vector>

#include "ecf8.h"
#include "ecf8_layout.h"

namespace {

using namespace ecf8;

// The reference rule on one 16-bit window W at a code start, packed as
// (v << 8) | len.  -1 when the rule leaves the LUT stack or yields a value
// above 15 (LUTs that ecf8_validate_format rejects).
int rule16(const uint8_t *luts, int n_luts, uint32_t w) {
  int v = luts[w >> 8];
  if (v >= 240) {
    const int row = 256 - v;
    if (row > n_luts - 2) return -1;
    v = luts[row * 256 + (w & 0xFF)];
  }
  if (v > 15) return -1;
  return (v << 8) | luts[(n_luts - 1) * 256 + v];
}

// Multi-symbol table.  A symbol is accepted only while the rule's result
// provably does not depend on the bits after the 12-bit window (every LUT
// entry the unknown bits could select holds the same value), so the table
// is exact for any LUT stack.
void build_multi(const uint8_t *luts, int n_luts, uint32_t *table) {
  const uint8_t *len_row = luts + 256 * (n_luts - 1);
  for (int w = 0; w < kMultiEntries; ++w) {
    uint32_t syms = 0, mask = 0;
    int n = 0, off = 0;
    while (n < kMaxSymsPerEntry && off < kWinBits) {
      const int known = kWinBits - off;  // window bits from this symbol's start
      const int kb = known < 8 ? known : 8;
      const int idx = ((w >> (known - kb)) & ((1 << kb) - 1)) << (8 - kb);
      const int span = 1 << (8 - kb);
      int v = luts[idx];
      bool fixed = true;
      for (int x = 1; x < span; ++x) fixed &= luts[idx + x] == v;
      if (!fixed) break;
      if (v >= 240) {
        const int row = 256 - v;
        if (row > n_luts - 2) break;
        const int known2 = known - 8;  // bits of the second byte inside the window
        const int kb2 = known2 <= 0 ? 0 : (known2 < 8 ? known2 : 8);
        const int idx2 = kb2 ? ((w >> (known2 - kb2)) & ((1 << kb2) - 1)) << (8 - kb2) : 0;
        const int span2 = 1 << (8 - kb2);
        const uint8_t *r = luts + 256 * row;
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
    table[w] = n ? (syms | (mask << 16) | ((uint32_t)off << 28)) : 0u;
  }
}

constexpr int kMixed = -2;

// Byte automaton.  `det[(1 << m) | q]` is the rule's result for every
// 16-bit window starting with the m-bit prefix q, or kMixed when windows
// with that prefix disagree.  A state is the bit string read since the
// current code start; it is pending while its rule result is mixed (or
// names a code longer than the bits read).  A symbol whose rule result is
// fixed only by bits past its own length (the LUT range of the EOF code,
// filled with the preceding symbol) "rewinds": decoding resumes inside the
// bits already read.  Chunks that reach a code-less entry, or more than 4
// symbols in one byte after a rewind, go to the exact row.  Returns false
// when the LUTs do not fit the automaton (more than 15 pending prefixes,
// more than 4 symbols in one byte without a rewind, i.e. a 1-bit code, or a
// rule result outside the stack).
class DfaBuilder {
 public:
  DfaBuilder(const uint8_t *luts, int n_luts) : det_(1u << 17), row_of_(1u << 16, -1) {
    for (uint32_t w = 0; w < 65536; ++w) det_[(1u << 16) | w] = rule16(luts, n_luts, w);
    for (int m = 15; m >= 0; --m) {
      for (uint32_t q = 0; q < (1u << m); ++q) {
        const int a = det_[(1u << (m + 1)) | (2 * q)];
        const int b = det_[(1u << (m + 1)) | (2 * q + 1)];
        det_[(1u << m) | q] = a == b ? a : kMixed;
      }
    }
  }

  bool build(uint32_t *table) {
    for (int b = 0; b < 256; ++b)
      if (!walk(1u, (uint32_t)b, 8, &table[b])) return false;
    for (int r = 1; r < 8; ++r)
      for (int b = 0; b < 256; ++b)
        if (!walk(1u, (uint32_t)b & ((1u << (8 - r)) - 1), 8 - r, &table[r * 256 + b]))
          return false;
    for (size_t i = 0; i < pending_.size(); ++i)  // grows while it is walked
      for (int b = 0; b < 256; ++b)
        if (!walk(pending_[i], (uint32_t)b, 8, &table[(kDfaFirstPendingRow + i) * 256 + b]))
          return false;
    const uint32_t exact = (uint32_t)kDfaExactRow << 10;
    for (int row = kDfaFirstPendingRow + (int)pending_.size(); row < kDfaRows; ++row)
      for (int b = 0; b < 256; ++b) table[row * 256 + b] = exact;  // never reached
    for (int b = 0; b < 256; ++b) table[kDfaExactRow * 256 + b] = exact;
    for (int r = 0; r < 8; ++r) table[kDfaSkipByte + r] = (uint32_t)r << 10;
    return true;
  }

 private:
  // Row of a pending prefix given as (1 << length) | bits; -1 when full.
  int intern(uint32_t key) {
    if (row_of_[key] >= 0) return row_of_[key];
    if ((int)pending_.size() == kDfaMaxPending) return -1;
    row_of_[key] = kDfaFirstPendingRow + (int)pending_.size();
    pending_.push_back(key);
    return row_of_[key];
  }

  // Decode `nbits` input bits after the pending prefix `pk`; write the entry.
  bool walk(uint32_t pk, uint32_t in, int nbits, uint32_t *entry) {
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
      const int r = det_[(1u << k) | q];
      if (r >= 0 && (r & 0xFF) > 16) return false;  // a length the format cannot hold
      if (r == kMixed || (r >= 0 && (r & 0xFF) > avail)) {
        // avail < 16 here: a 16-bit window always determines the rule
        next = intern((1u << avail) | (uint32_t)(t & ((1u << avail) - 1)));
        break;
      }
      if (r < 0) return false;
      const int l = r & 0xFF;
      if (l == 0) {  // code-less entry: the reference's decode of the chunk stops
        next = kDfaExactRow;
        break;
      }
      if (det_[(1u << l) | (q >> (k - l))] != r) rewound = true;
      if (count == kDfaMaxSyms) {
        if (!rewound) return false;
        next = kDfaExactRow;
        break;
      }
      syms |= (uint32_t)(r >> 8) << (4 * count);
      ++count;
      pos += l;
    }
    if (next < 0) return false;
    *entry = (uint32_t)(4 * count) | ((uint32_t)next << 10) | (syms << 16);
    return true;
  }

  std::vector<int> det_;
  std::vector<int> row_of_;
  std::vector<uint32_t> pending_;
};

}  // namespace

extern "C" int ecf8_build_table_host(const uint8_t *luts, int n_luts, int want_kind,
                                     uint32_t *table, int *table_kind) {
  if (!luts || !table) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  if (want_kind != ECF8_TABLE_ANY && want_kind != ECF8_TABLE_MULTI && want_kind != ECF8_TABLE_DFA)
    return ECF8_ERR_INVALID_ARG;
  memset(table, 0, ECF8_TABLE_BYTES);
  if (want_kind != ECF8_TABLE_MULTI) {
    DfaBuilder dfa(luts, n_luts);
    if (dfa.build(table)) {
      if (table_kind) *table_kind = ECF8_TABLE_DFA;
      return ECF8_OK;
    }
    if (want_kind == ECF8_TABLE_DFA) return ECF8_ERR_FORMAT;
    memset(table, 0, ECF8_TABLE_BYTES);
  }
  build_multi(luts, n_luts, table);
  if (table_kind) *table_kind = ECF8_TABLE_MULTI;
  return ECF8_OK;
}
