/*
 * CPU oracle for the ECF8 codec -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference's bitstream encoder
 * (dfloat/utils.py:373-499) and of its GPU decode rule
 * (dfloat/run/decode.cu:15-211), used by tests/ to check the HIP decoder at
 * sizes the pure-Python restatement cannot reach, and by bench.py as the
 * timed CPU baseline.  Nothing in the product links this file.
 */
#include <stdint.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_ERR_CAPACITY -1
#define ORACLE_ERR_ZERO_LENGTH -2
#define ORACLE_ERR_SYMBOL -3

/*
 * Encoder, following _encode_exponents_for_cuda (utils.py:373-499) step by
 * step: per symbol, record the chunk gap when a new chunk starts (:392-400),
 * the block output position when a new block starts (:405-406), append the
 * code MSB-first (:412-432); after the last symbol pad the final partial byte
 * with the leading bits of the EOF code (:439-459); close output_positions
 * with n (:463); zero-pad gaps to blocks*threads_per_block entries and pack
 * them 4 bits each, even chunk in the high nibble (:470-494).
 *
 * code_bits/code_vals are indexed by symbol 0..15 (bits == 0: symbol absent).
 * gaps_packed must hold ceil(n_bytes/(bpt*tpb))*tpb/2 bytes, encoded
 * ceil(sum bits/8) bytes, op (n_blocks+1) entries.
 */
int oracle_encode(const uint8_t *exps, int64_t n,
                  const uint8_t *code_bits, const uint32_t *code_vals,
                  int eof_bits, uint32_t eof_val,
                  int bytes_per_thread, int threads_per_block,
                  uint8_t *encoded, int64_t enc_cap, int64_t *n_bytes_out,
                  uint8_t *gaps_packed, int64_t gaps_cap, int64_t *gaps_bytes_out,
                  uint64_t *op, int64_t op_cap, int64_t *n_op_out,
                  uint8_t *gap_scratch, int64_t gap_scratch_cap)
{
    const int64_t bits_per_thread = 8LL * bytes_per_thread;
    const int64_t bits_per_block = bits_per_thread * threads_per_block;
    uint64_t buffer = 0;
    int size = 0;
    int64_t total_size = 0, element_count = 0;
    int64_t n_enc = 0, n_gaps = 0, n_op = 0;

    for (int64_t i = 0; i < n; i++) {
        const int s = exps[i];
        if (s > 15 || code_bits[s] == 0)
            return ORACLE_ERR_SYMBOL;
        if (total_size / bits_per_thread + 1 > n_gaps) {
            if (n_gaps >= gap_scratch_cap) return ORACLE_ERR_CAPACITY;
            gap_scratch[n_gaps++] = (uint8_t)(total_size % bits_per_thread);
        }
        if (total_size / bits_per_block + 1 > n_op) {
            if (n_op >= op_cap) return ORACLE_ERR_CAPACITY;
            op[n_op++] = (uint64_t)element_count;
        }
        const int bits = code_bits[s];
        buffer = (buffer << bits) + code_vals[s];
        size += bits;
        total_size += bits;
        element_count += 1;
        while (size >= 8) {
            const uint64_t byte = buffer >> (size - 8);
            if (n_enc >= enc_cap) return ORACLE_ERR_CAPACITY;
            encoded[n_enc++] = (uint8_t)byte;
            buffer -= byte << (size - 8);
            size -= 8;
        }
    }
    if (size > 0) {
        if (total_size / bits_per_thread + 1 > n_gaps) {
            if (n_gaps >= gap_scratch_cap) return ORACLE_ERR_CAPACITY;
            gap_scratch[n_gaps++] = (uint8_t)(total_size % bits_per_thread);
        }
        if (total_size / bits_per_block + 1 > n_op) {
            if (n_op >= op_cap) return ORACLE_ERR_CAPACITY;
            op[n_op++] = (uint64_t)element_count;
        }
        buffer = (buffer << eof_bits) + eof_val;
        size += eof_bits;
        const uint64_t byte = size >= 8 ? buffer >> (size - 8) : buffer << (8 - size);
        if (n_enc >= enc_cap) return ORACLE_ERR_CAPACITY;
        encoded[n_enc++] = (uint8_t)byte;
    }
    if (n_op >= op_cap) return ORACLE_ERR_CAPACITY;
    op[n_op++] = (uint64_t)n;

    const int64_t bytes_per_block = (int64_t)threads_per_block * bytes_per_thread;
    const int64_t blocks = (n_enc + bytes_per_block - 1) / bytes_per_block;
    const int64_t total_gaps = blocks * threads_per_block;
    if (total_gaps > gap_scratch_cap || total_gaps / 2 > gaps_cap) return ORACLE_ERR_CAPACITY;
    for (int64_t g = n_gaps; g < total_gaps; g++) gap_scratch[g] = 0;
    for (int64_t j = 0; j < total_gaps / 2; j++)
        gaps_packed[j] = (uint8_t)(((gap_scratch[2 * j] & 0xF) << 4) | (gap_scratch[2 * j + 1] & 0xF));

    *n_bytes_out = n_enc;
    *gaps_bytes_out = total_gaps / 2;
    *n_op_out = n_op;
    return ORACLE_OK;
}

/* One symbol from the next 16 bits, decode.cu:86-91. */
static inline int lut_decode_one(const uint8_t *luts, int n_luts, uint32_t w16, int *len)
{
    int v = luts[w16 >> 8];
    if (v >= 240) v = luts[256 * (256 - v) + (w16 & 0xFF)];
    *len = luts[256 * (n_luts - 1) + v];
    return v;
}

/*
 * Decode format-blocks [block_begin, block_end) of one compressed block
 * (decode.cu:15-211).  Chunk g owns the symbols starting at bit offsets
 * gap_g <= c < 8*bpt of its window (chunk plus 2 look-ahead bytes; bytes past
 * the stream read as 0).  The symbols of format-block b, in chunk order, go to
 * outputs[op[b] + k] for op[b] + k < min(op[b+1], n_elements); each output
 * byte merges the exponent with its sign/mantissa nibble (decode.cu:174-176).
 */
int oracle_decode_range(const uint8_t *luts, int n_luts,
                        const uint8_t *encoded, int64_t n_bytes,
                        const uint8_t *packed, const uint64_t *op,
                        const uint8_t *gaps, uint8_t *out, int64_t n_elements,
                        int threads_per_block, int bytes_per_thread,
                        int64_t block_begin, int64_t block_end)
{
    const int win_bytes = bytes_per_thread + 2;
    const int chunk_bits = 8 * bytes_per_thread;
    for (int64_t b = block_begin; b < block_end; b++) {
        int64_t idx = (int64_t)op[b];
        int64_t end = (int64_t)op[b + 1];
        if (end > n_elements) end = n_elements;
        for (int t = 0; t < threads_per_block && idx < end; t++) {
            const int64_t g = b * threads_per_block + t;
            /* the window as a big-endian bit string, at most 8*(8+2) bits */
            uint8_t win[64 + 2];
            for (int i = 0; i < win_bytes; i++) {
                const int64_t j = g * bytes_per_thread + i;
                win[i] = j < n_bytes ? encoded[j] : 0;
            }
            const uint8_t gb = gaps[g / 2];
            int pos = (g % 2 == 0) ? (gb >> 4) & 0xF : gb & 0xF;
            while (pos < chunk_bits && idx < end) {
                /* 16 bits starting at bit pos */
                uint32_t w = 0;
                for (int k = 0; k < 3; k++) {
                    const int bi = pos / 8 + k;
                    w = (w << 8) | (bi < win_bytes ? win[bi] : 0);
                }
                w = (w >> (8 - pos % 8)) & 0xFFFF;
                int len;
                const int v = lut_decode_one(luts, n_luts, w, &len);
                /* A code-less entry (length 0) is reachable only through the
                 * EOF pad bits after the last symbol; the reference would spin
                 * there, every later symbol is past n_elements anyway. */
                if (len == 0) break;
                const int o = (idx % 2 == 0) ? packed[idx / 2] >> 4 : packed[idx / 2] & 0xF;
                out[idx] = (uint8_t)(((o & 8) << 4) | (v << 3) | (o & 7));
                idx++;
                pos += len;
            }
        }
    }
    return ORACLE_OK;
}
