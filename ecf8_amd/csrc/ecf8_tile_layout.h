// ECF8-T, the tiled execution layout of one compressed FP8 Linear W[N, K]
// (N a multiple of 16, K of 128), shared by the host encoder
// (ecf8_tile_host.cpp) and the device kernels (ecf8_tile.hip).
//
// The block's Huffman code is kept; only the order of the symbols and the
// framing change, so that one wave decodes exactly the B operands of the
// MFMAs it runs.  Segment s = p * (K / 128) + kg holds the 2048 elements of
// the 16 x 128 tile (rows 16p.., columns 128kg..) in MFMA lane order: symbol
// 32 l + j is lane l's operand element m = tile_operand_elem(j), row
// 16p + (l & 15), column 128kg + c(m) with c(m) = 16 (l >> 4) + m for
// m < 16 and 64 + 16 (l >> 4) + (m - 16) for m >= 16 -- lane l's operands
// of v_mfma_f32_16x16x32_fp8_fp8 for the four K32 slices of the group, in
// the order the FP8 linear feeds them.  Within each run of 8 symbols the
// elements come in the order 0, 4, 1, 5, 2, 6, 3, 7: the lane's staged
// exponent dword then holds elements 0..3 in its even nibbles and 4..7 in
// its odd ones, and each nibble byte holds elements j and j + 4, so two
// shift-and-insert pairs place them straight into the operand's two dwords
// (no byte interleave).
//
//   stream  u8     segment s's codes (MSB-first, as the reference's
//                  bitstream) at byte seg_off[s], 4-byte aligned, then 16
//                  padding bytes after the last segment
//   seg_off u32[S+1]  byte offsets, seg_off[S] = end of the last segment
//   gaps    u32[S*8]  per 12-byte chunk c of a segment (c < 64), the bit
//                  offset of the first code starting in it (4 bits, chunk c
//                  in bits 4(c%8).. of word c/8)
//   other   u8[S*1024] sign/mantissa nibbles in the same order, two per
//                  byte, even symbol in the high nibble (the reference's
//                  packed_other_4bits convention)
//
// A segment occupies at most 64 chunks (768 bytes, 3 bits per element on
// average): the encoder refuses a Linear with a segment above that.
#ifndef ECF8_TILE_LAYOUT_H
#define ECF8_TILE_LAYOUT_H

#include <stdint.h>

namespace ecf8 {

constexpr int kTileRows = 16;
constexpr int kTileGroup = 128;
constexpr int kTileLanes = 64;
constexpr int kTileLaneSymbols = 32;
constexpr int kTileSegSymbols = kTileLanes * kTileLaneSymbols;  // 2048
constexpr int kTileChunkBytes = 12;
constexpr int kTileChunkBits = 8 * kTileChunkBytes;
constexpr int kTileMaxSegBytes = kTileLanes * kTileChunkBytes;  // 768
constexpr int kTileGapWords = kTileLanes / 8;                   // 8
constexpr int kTileOtherBytes = kTileSegSymbols / 2;            // 1024
constexpr int kTilePadBytes = 16;

// Operand element (0..31) of a lane's symbol j (0..31): runs of 8 in the
// order 0, 4, 1, 5, 2, 6, 3, 7.
constexpr int tile_operand_elem(int j) { return (j & ~7) | ((j & 1) << 2) | ((j & 7) >> 1); }

// Bytes a segment of `bits` code bits occupies (4-byte aligned).
inline int64_t tile_segment_bytes(int64_t bits) { return (((bits + 7) >> 3) + 3) & ~int64_t(3); }

}  // namespace ecf8

#endif  // ECF8_TILE_LAYOUT_H
