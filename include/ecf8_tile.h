/*
 * ecf8_tile.h -- the tiled execution layout ECF8-T of libecf8.so: one
 * compressed FP8 Linear re-encoded, under its block's own Huffman code, so
 * that the small-M linear of a decode step decodes its weight operands
 * itself instead of reading a decoded FP8 copy from HBM.
 *
 * No reference counterpart.  The reference decodes each block into FP8
 * before its GEMMs (dfloat/run/run.py:84-155, one decode per forward-pre-
 * hook); its on-disk layout (dfloat/utils.py:373-530) stays the checkpoint
 * format and the hook path's input, and a loader may re-tile a block's
 * Linears from it at load time (decode once, ecf8_tile_encode).
 *
 * Layout (N a multiple of 16, K of 128): segment s = p * (K/128) + kg holds
 * the 16 x 128 tile of rows 16p.., columns 128kg.. in MFMA lane order --
 * symbol 32 l + j is lane l's operand element m, row 16p + (l & 15),
 * column 128kg + 16 (l >> 4) + m (m < 16) or 128kg + 64 + 16 (l >> 4) +
 * (m - 16) (m >= 16), where m runs 0, 4, 1, 5, 2, 6, 3, 7 within each
 * run of 8 symbols (m = (j & ~7) | (j & 1) << 2 | (j & 7) >> 1): each
 * nibble byte then holds operand elements j and j + 4 of its run.
 *   stream   u8       each segment's codes, MSB-first, 4-byte aligned,
 *                     then 16 padding bytes
 *   seg_off  u32[S+1] segment byte offsets; seg_off[S] = end of the codes
 *   gaps     u32[8 S] bit offset of the first code in each 12-byte chunk
 *                     (4 bits per chunk, chunk c in bits 4(c%8) of word c/8)
 *   other    u8[1024 S] signs and mantissas, 4 bytes per run of 8
 *                     symbols: byte q of a run holds element q's mantissa
 *                     in bits 0..2 and sign in bit 7, element q + 4's
 *                     mantissa in bits 4..6, and in bit 3 the sign of
 *                     element ((q + 3) % 4) + 4 (FP8 bit positions, the
 *                     high elements' a 4-bit rotation of the dword away)
 * A segment holds at most 64 chunks (768 bytes).
 */
#ifndef ECF8_TILE_H
#define ECF8_TILE_H

#include <stdint.h>

#include "ecf8.h"
#include "ecf8_llm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ host */

/*
 * A Huffman code for the block's exponents recovered from its LUT stack:
 * for each exponent s of code length L (the stack's length row), the first
 * aligned block of 2^(16-L) 16-bit windows that the reference rule
 * (dfloat/run/decode.cu:85-91) decodes entirely to s gives code_bits[s] = L
 * and code_vals[s] = the block's L-bit prefix; code_bits[s] = 0 when no
 * such block exists.  Every code so recovered decodes to its symbol under
 * the rule (the compressor's own code, except where code-less windows of an
 * incomplete code form an earlier such block).  A window whose rule result
 * has code length 0 (the EOF code's range filled with an absent symbol)
 * carries no symbol; ECF8_ERR_FORMAT when a window leaves the LUT stack or
 * yields a value above 15 or a length above 16.
 */
int ecf8_code_from_luts(const uint8_t *luts, int n_luts, uint8_t *code_bits, uint32_t *code_vals);

/*
 * Sizes of the ECF8-T encoding of weight (e4m3fn bytes, row-major
 * [n_rows, k], host memory) under code_bits: stream bytes (padding
 * included) and segment count.  ECF8_ERR_CAPACITY when a segment exceeds
 * 768 bytes; ECF8_ERR_FORMAT when an exponent has no code.
 */
int ecf8_tile_sizes(const uint8_t *weight, int64_t n_rows, int64_t k, const uint8_t *code_bits,
                    int64_t *stream_bytes, int64_t *n_segments);

/*
 * Encode weight into the layout above (host memory; seg_off holds S+1
 * entries, gaps 8 S words, other 1024 S bytes), on up to n_threads host
 * threads.
 */
int ecf8_tile_encode(const uint8_t *weight, int64_t n_rows, int64_t k, const uint8_t *code_bits,
                     const uint32_t *code_vals, uint8_t *stream, int64_t stream_capacity,
                     uint32_t *seg_off, uint32_t *gaps, uint8_t *other, int n_threads);

/* ---------------------------------------------------------------- device */

/* One tiled weight operand (device memory) of a linear. */
typedef struct ecf8_tile_operand {
  const void *stream;        /* 4-byte aligned */
  const uint32_t *seg_off;
  const uint32_t *gaps;
  const void *other;         /* 16-byte aligned */
  const float *weight_scale; /* weight_scale_inv f32 [n/128, K/128] */
  int64_t n;                 /* output columns (rows of W), multiple of 128 */
  int64_t out_col;           /* first output column of this operand */
} ecf8_tile_operand;

/*
 * The small-M (M <= 16) block-scaled FP8 linear of ecf8_fp8_linear with
 * its weight operands decoded on the fly from ECF8-T:
 *   out[m, out_col + n] = sum_g (sum_{k in g} aq[m,k] W[n,k]) as[m,g] ws[n/128,g]
 * `table`: the ECF8_TABLE_DFA table of the block's LUTs (all operands
 * share the block's code).  `waves` (8 or 16) must be the wave count
 * ecf8_fp8_linear uses for the same shape -- 16 when K/128 >= 64, when
 * there are at most as many 16-column tiles as CUs, or when K = 4096 has
 * more than 2 x CUs tiles; else 8 -- and the result
 * is then bit-identical to decoding W and calling ecf8_fp8_linear.
 * aq: the tile layout of ecf8_llm.h (16-byte aligned, rows padded to 16);
 * out: bf16, ldo elements per row.
 */
int ecf8_tile_linear(const void *aq, const float *as, int64_t M, int64_t K,
                     const ecf8_tile_operand *ops, int n_ops, const uint32_t *table, void *out,
                     int64_t ldo, int waves, void *stream);

/*
 * Decode one tiled operand into row-major e4m3fn bytes out[n, K]
 * (16-byte aligned) with the DFA table of its block.
 */
int ecf8_tile_decode(const ecf8_tile_operand *op, int64_t K, const uint32_t *table, void *out,
                     void *stream);

/*
 * The grouped expert linear of ecf8_moe_linear (include/ecf8_llm.h) with
 * its weight operands decoded on the fly from ECF8-T, for a decode step of
 * M <= 16 routed tokens (so an expert holds at most 16 sorted pairs):
 *   out[q, s * seg_n + j] = linear(aq[row(q)], ops[e * n_segs + s])[j]
 * for every sorted position q of expert e.  ops: device array of
 * n_experts * n_segs operands (each [seg_n, K], its own out_col unused);
 * tables: device array of n_experts ECF8_TABLE_DFA tables (each expert's
 * block).  The wave count is ecf8_moe_linear's for this K (3 when K/128 =
 * 6, 8 when K/128 > ECF8_MOE_FOUR_WAVE_GROUPS, else 4), so the result is
 * bit-identical to
 * decoding the experts and calling ecf8_moe_linear.  Each routed expert's
 * 16-column tiles are dealt to its FP8 workgroups, every operand s getting
 * an equal run of them (so each wave reads one operand's addresses only):
 * splits > 0 FP8 workgroups per expert (rounded up for the runs), or,
 * splits = 0, one launch of the resident workgroups that the routed
 * experts share on the device (as many per expert as n_active leaves room
 * for), so that any routing runs in one round.  Idle workgroups exit, so
 * the launch can be captured in a graph.  The device arrays are trusted:
 * their pointers must satisfy ecf8_tile_linear's alignment rules.
 */
int ecf8_tile_moe_linear(const void *aq, const float *as, const int *row_of, const int *offsets,
                         const int *active, const int *n_active, int n_experts,
                         const ecf8_tile_operand *ops, const uint32_t *const *tables, int n_segs,
                         int64_t seg_n, int64_t K, int64_t M, void *out, int64_t ldo, int splits,
                         void *stream);

/*
 * ecf8_tile_decode over n_ops operands of one shape [n, K] in one launch:
 * ops, tables and outs are device arrays (operand i decodes with tables[i]
 * into outs[i], 16-byte aligned), e.g. one projection of every expert of a
 * layer.
 */
int ecf8_tile_decode_batch(const ecf8_tile_operand *ops, const uint32_t *const *tables,
                           void *const *outs, int n_ops, int64_t n, int64_t K, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ECF8_TILE_H */
