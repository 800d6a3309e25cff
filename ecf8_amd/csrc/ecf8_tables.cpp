// Host construction of the derived decode tables (layout in ecf8_layout.h)
// from a compressed block's LUT stack.  The steps are those of
// ecf8_table_build.h, run in loops; the device builder runs the same steps
// in parallel, so both give the same bytes.  Both tables reproduce the
// reference decode rule (dfloat/run/decode.cu:85-91) exactly; they are built
// once per compressed block, at load time, like the reference's
// shared_mem_size (dfloat/run/run.py:453-458).

#include <stdint.h>
#include <string.h>

#include <memory>

#include "ecf8.h"
#include "ecf8_layout.h"
#include "ecf8_table_build.h"

using namespace ecf8;

extern "C" int ecf8_build_table_host(const uint8_t *luts, int n_luts, int want_kind,
                                     uint32_t *table, int *table_kind) {
  if (!luts || !table) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  if (want_kind != ECF8_TABLE_ANY && want_kind != ECF8_TABLE_MULTI && want_kind != ECF8_TABLE_DFA)
    return ECF8_ERR_INVALID_ARG;
  std::unique_ptr<TableScratch> sp(new TableScratch());
  TableScratch &s = *sp;
  memcpy(s.luts, luts, (size_t)n_luts * 256);
  s.n_luts = n_luts;
  memset(table, 0, ECF8_TABLE_BYTES);
  if (want_kind != ECF8_TABLE_MULTI) {
    // range trees: the second-level rows, then the first level over their roots
    for (int t = 1; t <= second_level_rows(s); ++t) {
      for (int i = 0; i < 256; ++i) s.tree[t][256 + i] = tree_leaf(s, t, i);
      for (int n = 255; n >= 1; --n) s.tree[t][n] = tree_combine(s.tree[t][2 * n], s.tree[t][2 * n + 1]);
    }
    for (int i = 0; i < 256; ++i) s.tree[0][256 + i] = tree_leaf(s, 0, i);
    for (int n = 255; n >= 1; --n) s.tree[0][n] = tree_combine(s.tree[0][2 * n], s.tree[0][2 * n + 1]);
    // pending prefixes in canonical order (length, then bits)
    bool fits = true;
    s.n_pending = 0;
    for (int i = 0; i < kPrefixKeys && fits; ++i) {
      const uint32_t key = prefix_key(i);
      if (!prefix_pending(s, key)) continue;
      if (s.n_pending == kDfaMaxPending) fits = false;
      else s.pending[s.n_pending++] = key;
    }
    for (int e = 0; e < kDfaEntries && fits; ++e) fits = dfa_table_entry(s, e, &table[e]);
    if (fits) {
      table[kKindWord] = ECF8_TABLE_DFA;
      if (table_kind) *table_kind = ECF8_TABLE_DFA;
      return ECF8_OK;
    }
    if (want_kind == ECF8_TABLE_DFA) return ECF8_ERR_FORMAT;
    memset(table, 0, ECF8_TABLE_BYTES);
  }
  for (int w = 0; w < kMultiEntries; ++w) table[w] = multi_entry(s, w);
  table[kKindWord] = ECF8_TABLE_MULTI;
  if (table_kind) *table_kind = ECF8_TABLE_MULTI;
  return ECF8_OK;
}
