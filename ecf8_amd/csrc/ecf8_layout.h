// Layout of the derived decode tables, shared by the host builders
// (ecf8_tables.cpp) and the gfx950 decode kernels (ecf8_decode.hip).
//
// Both tables are derived from a block's on-disk LUT stack and reproduce the
// reference decode rule (dfloat/run/decode.cu:85-91):
//   v = L0[W >> 8];  if (v >= 240) v = L[256 - v][W & 0xFF];  len = Llen[v]
// where W is the 16-bit window at a code start.
#ifndef ECF8_LAYOUT_H
#define ECF8_LAYOUT_H

#include <stdint.h>

#if defined(__HIP__)
#define ECF8_HD __host__ __device__
#else
#define ECF8_HD
#endif

namespace ecf8 {

constexpr int kChunkBytes = 8;  // bytes_per_thread of the format
constexpr int kChunkBits = 8 * kChunkBytes;

// ---------------------------------------------------------------- multi
// ECF8_TABLE_MULTI: u32[4096] indexed by a 12-bit window at a code start.
//   bits  0..15  up to 4 exponents, first decoded in bits 0..3
//   bits 16..27  start mask: bit j set iff one of those symbols starts at
//                window offset j (so popcount = number of symbols)
//   bits 28..31  total code length of those symbols (0 = no symbol fully
//                determined by the 12 window bits)
constexpr int kWinBits = 12;
constexpr int kMultiEntries = 1 << kWinBits;
constexpr int kMaxSymsPerEntry = 4;
ECF8_HD constexpr uint32_t entry_len(uint32_t e) { return e >> 28; }
ECF8_HD constexpr uint32_t entry_mask(uint32_t e) { return (e >> 16) & 0xFFFu; }

// ------------------------------------------------------------------ dfa
// ECF8_TABLE_DFA: a byte automaton.  Row r (256 u32 entries, one per input
// byte) is a decoder state:
//   row 0            at a code start
//   rows 1..7        at a code start after skipping the next r bits (a
//                    chunk whose first code starts inside its first byte)
//   row 8            exact: the rest of the chunk is not expressible in
//                    this table (a code-less LUT entry, or more than 4
//                    symbols in one byte after a LUT entry that consumes
//                    fewer bits than it reads -- both only where EOF bits
//                    are read, i.e. in the stream's final padding); the
//                    kernel decodes such a chunk with the LUT rule itself
//   rows 9..23       inside a code: the bits read since the code start are
//                    a prefix that does not yet determine the symbol
// followed by 8 "skip a whole byte" entries (index 24*256 + r) that move to
// row r without decoding, for chunks whose first code starts in byte 1.
// Entry layout:
//   bits  0..7   4 x the number of symbols completed in this byte (0..16:
//                their width in bits of packed nibbles; a whole byte, so it
//                can be added without a mask)
//   bits 10..14  next row (so entry & kDfaRowMask = next row * 1024 = the
//                byte offset of that row in the table)
//   bits 16..31  the completed symbols' exponents, first in bits 16..19;
//                unused nibbles are zero
constexpr int kDfaRows = 24;
constexpr int kDfaExactRow = 8;
constexpr int kDfaFirstPendingRow = 9;
constexpr int kDfaMaxPending = kDfaRows - kDfaFirstPendingRow;  // 15
constexpr int kDfaSkipByte = kDfaRows * 256;                      // entry index
constexpr int kDfaEntries = kDfaSkipByte + 8;                     // 6152
constexpr uint32_t kDfaRowMask = 0x7C00u;
constexpr int kDfaMaxSyms = 4;

}  // namespace ecf8

#endif  // ECF8_LAYOUT_H
