// Host side of the tiled execution layout (ECF8-T; layout in
// ecf8_tile_layout.h): recovering a block's Huffman code from its LUT stack,
// and re-encoding one FP8 Linear into MFMA-order segments under that code.
// No reference counterpart: the reference decodes each block into FP8
// before its GEMM (dfloat/run/run.py:84-155); this layout lets the small-M
// linear decode the exponents itself (ecf8_tile_linear), with the block's
// own code, so the compressed size is the reference layout's.

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "ecf8.h"
#include "ecf8_tile.h"
#include "ecf8_tile_layout.h"

using namespace ecf8;

namespace {

// Element (row, column) of symbol i of segment (panel p, group kg): lane
// i / 32's operand element m = tile_operand_elem(i % 32).
inline void tile_element(int64_t p, int64_t kg, int i, int64_t *row, int64_t *col) {
  const int lane = i / kTileLaneSymbols, m = tile_operand_elem(i % kTileLaneSymbols);
  const int r = lane & 15, q = lane >> 4;
  *row = p * kTileRows + r;
  *col = kg * kTileGroup + (m < 16 ? 16 * q + m : 64 + 16 * q + (m - 16));
}

inline int exponent_of(uint8_t b) { return (b >> 3) & 0xF; }

// Sign and mantissa of symbol i into the segment's nibble plane: each run
// of 8 symbols (operand elements q and q + 4 at symbols 2q and 2q + 1) owns
// 4 bytes; byte q holds element q's mantissa in bits 0..2 and sign in bit
// 7, element q + 4's mantissa in bits 4..6, and in bit 3 the sign of
// element ((q + 3) % 4) + 4 -- so that a 4-bit rotation of the run's dword
// puts every high element's sign and mantissa where its FP8 byte has them.
inline void put_sign_mantissa(uint8_t *other, int i, uint8_t b) {
  uint8_t *const run = other + (i >> 3) * 4;
  const int q = (i & 7) >> 1, sign = b >> 7, mant = b & 7;
  if (!(i & 1)) {
    run[q] |= (uint8_t)(mant | sign << 7);
  } else {
    run[q] |= (uint8_t)(mant << 4);
    run[(q + 1) & 3] |= (uint8_t)(sign << 3);
  }
}

// Bits of one segment under the code lengths.
int64_t segment_bits(const uint8_t *w, int64_t k, int64_t p, int64_t kg, const uint8_t *code_bits,
                     bool *missing) {
  int64_t bits = 0;
  for (int i = 0; i < kTileSegSymbols; ++i) {
    int64_t row, col;
    tile_element(p, kg, i, &row, &col);
    const int e = exponent_of(w[row * k + col]);
    if (code_bits[e] == 0) *missing = true;
    bits += code_bits[e];
  }
  return bits;
}

// Write one segment: codes MSB-first from the segment's first byte, chunk
// gaps, sign/mantissa nibbles.  `out` holds the segment's bytes (zeroed).
void write_segment(const uint8_t *w, int64_t k, int64_t p, int64_t kg, const uint8_t *code_bits,
                   const uint32_t *code_vals, uint8_t *out, uint32_t *gaps, uint8_t *other) {
  uint64_t acc = 0;  // pending bits, right-aligned
  int nacc = 0;
  int64_t nbyte = 0, pos = 0;
  int next_chunk = 0;  // first chunk whose gap is not yet recorded
  memset(gaps, 0, kTileGapWords * 4);
  memset(other, 0, kTileOtherBytes);
  for (int i = 0; i < kTileSegSymbols; ++i) {
    int64_t row, col;
    tile_element(p, kg, i, &row, &col);
    const uint8_t b = w[row * k + col];
    const int e = exponent_of(b), len = code_bits[e];
    // the first code starting in each chunk: its offset in the chunk
    while (next_chunk < kTileLanes && pos >= (int64_t)next_chunk * kTileChunkBits) {
      const int64_t gap = pos - (int64_t)next_chunk * kTileChunkBits;
      if (gap < kTileChunkBits) gaps[next_chunk >> 3] |= (uint32_t)gap << (4 * (next_chunk & 7));
      ++next_chunk;
    }
    acc = (acc << len) | code_vals[e];
    nacc += len;
    pos += len;
    while (nacc >= 8) {
      out[nbyte++] = (uint8_t)(acc >> (nacc - 8));
      nacc -= 8;
    }
    put_sign_mantissa(other, i, b);
  }
  if (nacc) out[nbyte++] = (uint8_t)(acc << (8 - nacc));
}

}  // namespace

extern "C" int ecf8_code_from_luts(const uint8_t *luts, int n_luts, uint8_t *code_bits,
                                   uint32_t *code_vals) {
  if (!luts || !code_bits || !code_vals) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  const uint8_t *len_row = luts + 256 * (n_luts - 1);
  memset(code_bits, 0, 16);
  memset(code_vals, 0, 16 * sizeof(uint32_t));
  // the symbol every 16-bit window decodes to under the reference rule
  // (dfloat/run/decode.cu:85-91); kNoSymbol for a window whose result has no
  // code (length 0): the LUT builder fills the range of the EOF code with
  // the symbol before it, or with 0 when the EOF code is the lowest key --
  // such windows only occur in a stream's final padding
  constexpr uint8_t kNoSymbol = 0xFF;
  std::vector<uint8_t> sym(65536);
  for (uint32_t w = 0; w < 65536; ++w) {
    int v = luts[w >> 8];
    if (v >= 240) {
      const int row = 256 - v;
      if (row > n_luts - 2) return ECF8_ERR_FORMAT;
      v = luts[row * 256 + (w & 0xFF)];
    }
    if (v > 15) return ECF8_ERR_FORMAT;
    const int len = len_row[v];
    if (len > 16) return ECF8_ERR_FORMAT;
    sym[w] = len ? (uint8_t)v : kNoSymbol;
  }
  // A symbol's code of length L: the first aligned block of 2^(16-L)
  // windows that all decode to it.  The rule decodes every window of such a
  // block to the symbol and consumes L bits, so the block encodes the
  // symbol whether or not it is the compressor's own code -- an incomplete
  // code (Kraft sum below 1) leaves code-less windows that the LUT builder
  // fills with some symbol, so "the first window decoding to s" is not a
  // code in general.
  for (int s = 0; s < 16; ++s) {
    const int len = len_row[s];
    if (len < 1 || len > 16) continue;
    const uint32_t span = 1u << (16 - len);
    for (uint32_t lo = 0; lo < 65536; lo += span) {
      bool all = true;
      for (uint32_t w = lo; w < lo + span && all; ++w) all = sym[w] == s;
      if (all) {
        code_bits[s] = (uint8_t)len;
        code_vals[s] = lo >> (16 - len);
        break;
      }
    }
  }
  return ECF8_OK;
}

extern "C" int ecf8_tile_sizes(const uint8_t *weight, int64_t n_rows, int64_t k,
                               const uint8_t *code_bits, int64_t *stream_bytes,
                               int64_t *n_segments) {
  if (!weight || !code_bits || !stream_bytes || !n_segments || n_rows <= 0 || k <= 0)
    return ECF8_ERR_INVALID_ARG;
  if (n_rows % kTileRows || k % kTileGroup) return ECF8_ERR_UNSUPPORTED;
  const int64_t panels = n_rows / kTileRows, groups = k / kTileGroup;
  int64_t total = 0;
  bool missing = false;
  for (int64_t p = 0; p < panels; ++p) {
    for (int64_t kg = 0; kg < groups; ++kg) {
      const int64_t bytes = tile_segment_bytes(segment_bits(weight, k, p, kg, code_bits, &missing));
      if (bytes > kTileMaxSegBytes) return ECF8_ERR_CAPACITY;
      total += bytes;
    }
  }
  if (missing) return ECF8_ERR_FORMAT;  // an exponent without a code
  if (total + kTilePadBytes > (int64_t)UINT32_MAX) return ECF8_ERR_UNSUPPORTED;
  *stream_bytes = total + kTilePadBytes;
  *n_segments = panels * groups;
  return ECF8_OK;
}

extern "C" int ecf8_tile_encode(const uint8_t *weight, int64_t n_rows, int64_t k,
                                const uint8_t *code_bits, const uint32_t *code_vals,
                                uint8_t *stream, int64_t stream_capacity, uint32_t *seg_off,
                                uint32_t *gaps, uint8_t *other, int n_threads) {
  if (!weight || !code_bits || !code_vals || !stream || !seg_off || !gaps || !other ||
      n_rows <= 0 || k <= 0)
    return ECF8_ERR_INVALID_ARG;
  if (n_rows % kTileRows || k % kTileGroup) return ECF8_ERR_UNSUPPORTED;
  for (int s = 0; s < 16; ++s)
    if (code_bits[s] > 16 || (code_bits[s] && code_vals[s] >> code_bits[s])) return ECF8_ERR_FORMAT;
  const int64_t panels = n_rows / kTileRows, groups = k / kTileGroup, n_seg = panels * groups;
  const int nt = std::max(1, std::min(n_threads, 64));
  // pass 1: segment sizes (parallel), then offsets
  std::vector<int64_t> bytes(n_seg);
  std::vector<int> bad(nt, 0);
  auto run = [&](auto &&body) {
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t)
      th.emplace_back([&, t] {
        for (int64_t s = t; s < n_seg; s += nt) body(t, s);
      });
    for (auto &x : th) x.join();
  };
  run([&](int t, int64_t s) {
    bool missing = false;
    bytes[s] = tile_segment_bytes(segment_bits(weight, k, s / groups, s % groups, code_bits,
                                               &missing));
    if (missing) bad[t] |= 1;
    if (bytes[s] > kTileMaxSegBytes) bad[t] |= 2;
  });
  int any_bad = 0;
  for (int b : bad) any_bad |= b;
  if (any_bad & 1) return ECF8_ERR_FORMAT;
  if (any_bad & 2) return ECF8_ERR_CAPACITY;
  int64_t off = 0;
  for (int64_t s = 0; s < n_seg; ++s) {
    if (off > (int64_t)UINT32_MAX) return ECF8_ERR_UNSUPPORTED;
    seg_off[s] = (uint32_t)off;
    off += bytes[s];
  }
  if (off + kTilePadBytes > stream_capacity || off > (int64_t)UINT32_MAX) return ECF8_ERR_CAPACITY;
  seg_off[n_seg] = (uint32_t)off;
  memset(stream, 0, (size_t)(off + kTilePadBytes));
  // pass 2: the segments (parallel; disjoint outputs)
  run([&](int, int64_t s) {
    write_segment(weight, k, s / groups, s % groups, code_bits, code_vals, stream + seg_off[s],
                  gaps + s * kTileGapWords, other + s * kTileOtherBytes);
  });
  return ECF8_OK;
}
