/*
 * ecf8.h -- C ABI of libecf8.so, the MI355X (gfx950) ECF8 decode engine.
 *
 * Plain pointers and sizes only.  Device pointers are HIP device addresses
 * (e.g. torch tensor data_ptr()); `stream` is a hipStream_t passed as void*
 * (NULL = the null stream).  Every call returns an ECF8_* status; device
 * calls are asynchronous on `stream` and allocate nothing.
 *
 * Reference interfaces each entry point replaces are cited as
 * file:line of zeyuyang8/ecf8.
 */
#ifndef ECF8_H
#define ECF8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ECF8_OK 0
#define ECF8_ERR_INVALID_ARG 1       /* null pointer, negative size, odd n     */
#define ECF8_ERR_UNSUPPORTED 2       /* format geometry the kernels do not run */
#define ECF8_ERR_MISALIGNED 3        /* device buffer alignment not met        */
#define ECF8_ERR_FORMAT 4            /* compressed block fails validation      */
#define ECF8_ERR_HIP 5               /* HIP runtime error (launch, device)     */
#define ECF8_ERR_CAPACITY 6          /* caller buffer too small                */

/* Bytes of a derived decode table buffer (either kind): the table's entries,
 * then at u32 index 6152 the kind it holds (ECF8_TABLE_DFA or
 * ECF8_TABLE_MULTI), then zero padding. */
#define ECF8_TABLE_BYTES 24624
/* Kinds of derived decode table. */
#define ECF8_TABLE_ANY (-1)   /* builder's choice: DFA when the LUTs allow it */
#define ECF8_TABLE_MULTI 0    /* 12-bit multi-symbol table; any LUT stack      */
#define ECF8_TABLE_DFA 1      /* byte automaton; prefix-code LUTs with <= 15
                                 pending prefixes and <= 4 codes per byte     */
/* Largest LUT stack the format allows: 1 first-level row, at most 16
 * second-level rows (pointer values 240..255, dfloat/run/decode.cu:87),
 * 1 length row. */
#define ECF8_MAX_LUTS 18

const char *ecf8_version(void);
const char *ecf8_status_string(int status);

/* ---------------------------------------------------------------- device */

/*
 * Build the derived decode table from a block's on-disk LUTs.
 * No reference counterpart: the reference walks the LUTs per symbol
 * (dfloat/run/decode.cu:86-91); the table is computed once per compressed
 * block (at load time, like shared_mem_size in dfloat/run/run.py:453-458) and
 * reproduces the reference's rule exactly.  Two kinds:
 *   ECF8_TABLE_DFA    a byte automaton (8-9 lookups per 8-byte chunk);
 *                     requires LUTs forming a prefix code with at most 15
 *                     pending prefixes and at most 4 codes ending in any
 *                     byte (every code >= 2 bits)
 *   ECF8_TABLE_MULTI  12-bit windows, up to 4 symbols per lookup; any LUTs
 * want_kind ECF8_TABLE_ANY picks DFA when possible; asking for DFA when it
 * is not possible returns ECF8_ERR_FORMAT.  *table_kind receives the kind
 * built; pass it to ecf8_decode.  The automaton's pending rows are numbered
 * in a canonical order (prefix length, then bits), so both builders write
 * the same bytes for the same LUTs.
 *
 * ecf8_build_table_host: luts and table in host memory
 *   (table: ECF8_TABLE_BYTES).
 * ecf8_build_table: luts (4-byte aligned) and table (ECF8_TABLE_BYTES,
 *   4-byte aligned) in device memory, built by one workgroup on `stream`.
 *   table_kind NULL: fully asynchronous (no host round trip, capturable in
 *   a HIP graph); the kind is then only known on the device, so pass
 *   ECF8_TABLE_ANY to ecf8_decode.  want_kind ECF8_TABLE_DFA requires a
 *   non-NULL table_kind.  table_kind non-NULL: the kind word is copied back
 *   and `stream` synchronized.
 */
int ecf8_build_table_host(const uint8_t *luts, int n_luts, int want_kind, uint32_t *table,
                          int *table_kind);
int ecf8_build_table(const uint8_t *luts, int n_luts, int want_kind, uint32_t *table,
                     int *table_kind, void *stream);

/*
 * The derived table of `luts`, kept in a caller-owned device buffer `cache`
 * of ECF8_TABLE_CACHE_BYTES (8-byte aligned): the table (its first
 * ECF8_TABLE_BYTES, the `table` argument of ecf8_decode), then the LUT
 * bytes and want_kind it was built from.  One workgroup on `stream`
 * compares the LUTs with that copy and rebuilds the table (as
 * ecf8_build_table with a NULL table_kind) only when they differ; a
 * zero-filled cache never matches.  Fully asynchronous and capturable.
 * No reference counterpart: it makes the reference's per-call decode form
 * (the RawKernel launch of dfloat/run/run.py:104-119, which a call-form
 * stand-in must serve without knowing whether the LUTs changed since the
 * last call) cost a compare of at most 4,608 bytes instead of a rebuild.
 * Calls sharing one cache must not overlap (one stream per cache).
 */
#define ECF8_TABLE_CACHE_BYTES (ECF8_TABLE_BYTES + 8 + ECF8_MAX_LUTS * 256)
int ecf8_build_table_cached(const uint8_t *luts, int n_luts, int want_kind, void *cache,
                            void *stream);

/*
 * Decode one compressed block into FP8 e4m3fn bytes.
 * Replaces the CUDA kernel `decode` (dfloat/run/decode.cu:15-26) as launched
 * by decode_hook (dfloat/run/run.py:97-119) and validate_cuda_decoding_fp8
 * (scripts/compress.py:86-124).  Arguments keep the reference's meaning:
 *   luts               device u8[n_luts*256]   (run.py:109)
 *   encoded            device u8[n_bytes]      (run.py:110), 16-byte aligned
 *   packed_other_4bits device u8[n_elements/2] (run.py:111), 8-byte aligned
 *   output_positions   device u64[n_fb+1]      (run.py:112)
 *   gaps               device u8[n_fb*threads_per_block/2] (run.py:113)
 *   outputs            device u8[n_elements]   (run.py:114), 16-byte aligned
 *   table, table_kind  the derived table ecf8_build_table built for these
 *                      luts, and its kind; ECF8_TABLE_ANY reads the kind
 *                      from the table on the device (both decode kernels
 *                      are launched and the one the table is not for exits
 *                      at once), so no host round trip is needed
 *   max_block_elements largest output_positions[b+1] - output_positions[b]
 *                      (the reference derives shared_mem_size from it,
 *                      dfloat/run/run.py:453-458); sizes the kernel's LDS
 *                      staging.  0 = unknown (worst case is assumed).  A
 *                      value below the true maximum leaves the excess
 *                      elements of such blocks unwritten.
 *   min_code_bits      shortest nonzero code length in the LUTs' length row
 *                      (ecf8 length row = last LUT row); sizes the per-lane
 *                      LDS run of the ECF8_TABLE_MULTI kernel.  0 = unknown
 *                      (1 bit assumed).  A value above the true minimum can
 *                      leave outputs wrong, never touches memory out of
 *                      bounds.
 * where n_fb = ceil(n_bytes / (threads_per_block*bytes_per_thread)).
 * Geometry: bytes_per_thread must be 8 (the reference kernel hard-codes it,
 * decode.cu:5); threads_per_block one of 128, 256, 512, 1024.
 * Outputs outside [0, n_elements) are never written.  n_bytes and n_elements
 * must stay below 2^31 - 64 (the reference's positions are 32-bit,
 * decode.cu:23-25).
 */
int ecf8_decode(const uint8_t *luts, const uint8_t *encoded, const uint8_t *packed_other_4bits,
                const uint64_t *output_positions, const uint8_t *gaps, uint8_t *outputs,
                int n_luts, int64_t n_bytes, int64_t n_elements, int64_t max_block_elements,
                int min_code_bits, const uint32_t *table, int table_kind,
                int threads_per_block, int bytes_per_thread, void *stream);

/*
 * ecf8_decode with the reference kernel's arguments only, allocating
 * nothing and taking no workspace.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * derived table is built on `stream` into the library's static device
 * array (ECF8_TABLE_BYTES per GPU, held until the process ends), and the
 * decode reads its kind there.  Arguments, alignment and errors are those of
 * ecf8_decode (min_code_bits is taken as unknown); every argument error is
 * returned before any HIP call.  No input size can exceed the array: it
 * always holds one table.  Calls that overlap on one GPU (several streams
 * or host threads) race on that table; serialize them.
 */
int ecf8_decode_noalloc(const uint8_t *luts, const uint8_t *encoded,
                        const uint8_t *packed_other_4bits, const uint64_t *output_positions,
                        const uint8_t *gaps, uint8_t *outputs, int n_luts, int64_t n_bytes,
                        int64_t n_elements, int64_t max_block_elements, int threads_per_block,
                        int bytes_per_thread, void *stream);

/*
 * One compressed block of a batched decode.  The array of descriptors lives
 * in device memory; every field keeps its ecf8_decode meaning and
 * requirements (bytes_per_thread 8; `table` must be an ECF8_TABLE_DFA table
 * built for `luts`); blocks with fewer than 12 bitstream bytes or 16
 * elements are skipped (decode those with ecf8_decode).  task_begin is the
 * index of the block's first task:
 * task_begin[0] = 0 and task_begin[d+1] = task_begin[d] +
 * ceil(ceil(n_bytes[d] / (threads_per_block * 8)) / blocks_per_task).
 */
typedef struct ecf8_block_desc {
  const uint8_t *luts;
  const uint8_t *encoded;
  const uint8_t *packed_other_4bits;
  const uint64_t *output_positions;
  const uint8_t *gaps;
  uint8_t *outputs;
  const uint32_t *table;
  int64_t n_bytes;
  int64_t n_elements;
  int32_t n_luts;
  int32_t task_begin;
} ecf8_block_desc; /* 80 bytes */

/*
 * Decode many compressed blocks in one launch: the routed experts of an MoE
 * layer, or every block of a model.  No reference counterpart: the reference
 * launches `decode` once per block from each module's hook
 * (dfloat/run/run.py:97-119, per expert under the qwen3moe pattern of
 * dfloat/const.py:15-21).  The work is cut into tasks of up to
 * blocks_per_task format-blocks of one block (a block's tasks interleave
 * its format-blocks); n_tasks is the total.  max_block_elements bounds every block's largest format-block (0 =
 * unknown).  descs: device memory, 8-byte aligned.  Asynchronous on stream.
 */
int ecf8_decode_batched(const ecf8_block_desc *descs, int count, int n_tasks, int blocks_per_task,
                        int64_t max_block_elements, int threads_per_block, void *stream);

/*
 * Batched decode of the blocks whose select[d] (device int32, one per
 * descriptor) is nonzero, e.g. the attention block and the experts the
 * router picked for this step: the reference decodes only the experts whose
 * modules run (their hooks, dfloat/run/run.py:84-155).  Up to 256
 * descriptors (e.g. an MoE layer's attention block and 128 experts), one
 * launch: each workgroup of the batched kernel scans the flags itself and
 * workgroup 0 writes {selected count, their tasks} to work_counts (device
 * int32[2]); work_descs is not used.  More descriptors: a one-workgroup
 * kernel first compacts the selected ones into work_descs (device, `count`
 * entries) and writes the same two counts to work_counts, where the batched
 * kernel reads them.  Nothing is read back to the host, so the call can be
 * captured in a HIP graph and replayed with new flags.  descs' task_begin
 * fields are ignored.  Unselected blocks' outputs are not touched.
 */
int ecf8_decode_batched_select(const ecf8_block_desc *descs, int count, const int32_t *select,
                               ecf8_block_desc *work_descs, int32_t *work_counts,
                               int blocks_per_task, int64_t max_block_elements,
                               int threads_per_block, void *stream);

/*
 * One Linear of a compressed block for ecf8_decode_bf16: elements
 * [start, start + rows * cols) of the block's flat output are its row-major
 * weight [rows, cols] (start = the block's split_positions entry,
 * dfloat/utils.py:188-204), and `scale` its f32 block scales
 * [rows / 128][cols / 128] (device memory, row-major, 4-byte aligned).
 */
typedef struct ecf8_scaled_part {
  const float *scale;
  int64_t start;
  int64_t rows;
  int64_t cols;
} ecf8_scaled_part; /* 32 bytes */

#define ECF8_MAX_SCALED_PARTS 16

/*
 * Decode one compressed block straight into the bf16 weights its FP8
 * Linears compute with: output element q of part p is
 * bf16(fp8(q) * p.scale[r / 128][c / 128]) (r, c = q's row and column in
 * the part; f32 product, round to nearest even) -- the bytes that
 * ecf8_decode followed by ecf8_dequant_fp8_block on each part's view give,
 * in one pass that never writes the FP8 bytes.  No reference counterpart:
 * the reference decodes FP8 (dfloat/run/decode.cu:15-26) and its consumer
 * converts each Linear's weight per call; this serves consumers that run a
 * bf16 GEMM on block-scaled FP8 weights (the DiT flow, whose reference
 * hook is dfloat/run/run.py:84-155).
 * Arguments as ecf8_decode, with outputs replaced by out_bf16 (device
 * u16[n_elements], 16-byte aligned), and:
 *   table_kind  must be ECF8_TABLE_DFA (ECF8_ERR_UNSUPPORTED otherwise:
 *               decode with ecf8_decode and dequantize)
 *   parts       host array of n_parts (1..ECF8_MAX_SCALED_PARTS) parts in
 *               element order: parts[0].start = 0, each next start = the
 *               previous start + rows * cols, the last part ending at
 *               n_elements; rows and cols positive multiples of 128
 *   threads_per_block must be 512, bytes_per_thread 8; the block needs at
 *   least 12 bitstream bytes (ECF8_ERR_UNSUPPORTED otherwise).
 * Every argument error is returned before anything is launched.
 */
int ecf8_decode_bf16(const uint8_t *luts, const uint8_t *encoded,
                     const uint8_t *packed_other_4bits, const uint64_t *output_positions,
                     const uint8_t *gaps, uint16_t *out_bf16, int n_luts, int64_t n_bytes,
                     int64_t n_elements, int64_t max_block_elements, const uint32_t *table,
                     int table_kind, const ecf8_scaled_part *parts, int n_parts,
                     int threads_per_block, int bytes_per_thread, void *stream);

/* --------------------------------------------------------- measurement */

/*
 * Streaming probe for the bandwidth a one-launch kernel reaches on this
 * GPU (bench.py --mode ceiling): op 0 reads `bytes` of src (16-byte
 * aligned, a multiple of 16), op 1 copies them to dst; `grid` workgroups
 * of `block` (64..1024, a power of two) lanes sweep the buffer
 * grid-stride, each lane keeping `depth` (1, 2, 4 or 8) 16-byte loads in
 * flight, with non-temporal loads and stores if `nontemporal`.  `sink`: one
 * device u32 the read sweep may write.  No reference counterpart; the
 * decode path never calls it.
 */
int ecf8_stream_probe(int op, const void *src, void *dst, int64_t bytes, int grid, int block,
                      int depth, int nontemporal, uint32_t *sink, void *stream);

/* ------------------------------------------------------------------ host */

/*
 * Sizes of the encoder outputs for `n` exponents under the given code
 * lengths (code_bits[s] = length of symbol s, 0 = absent): encoded bytes,
 * packed gap bytes and output_positions entries.  Host memory.
 */
int ecf8_encoded_sizes(const uint8_t *exponents, int64_t n, const uint8_t *code_bits,
                       int bytes_per_thread, int threads_per_block,
                       int64_t *n_bytes, int64_t *gaps_bytes, int64_t *n_output_positions);

/*
 * Bitstream encoder.  Replaces _encode_exponents_for_cuda
 * (dfloat/utils.py:373-499) and encode_exponents_for_cuda (:502-530):
 * MSB-first Huffman codes, 4-bit per-chunk gaps (even chunk in the high
 * nibble), per-format-block output positions closed by n, final byte padded
 * with the leading bits of the EOF code.  code_bits/code_vals are indexed by
 * symbol 0..15; eof_bits/eof_value is the EOF pseudo-symbol's code.
 * Host memory; capacities from ecf8_encoded_sizes.
 */
int ecf8_encode_exponents(const uint8_t *exponents, int64_t n, const uint8_t *code_bits,
                          const uint32_t *code_vals, int eof_bits, uint32_t eof_value,
                          int bytes_per_thread, int threads_per_block,
                          uint8_t *encoded, int64_t encoded_capacity,
                          uint8_t *gaps, int64_t gaps_capacity,
                          uint64_t *output_positions, int64_t output_positions_capacity);

/*
 * Format validator for one compressed block (host memory).  No reference
 * counterpart (the reference validates nothing before launch); it checks the
 * invariants the decode rule relies on: LUT stack shape and pointers
 * (utils.py:270-370), n_luts <= 18, code lengths 1..16, gaps/output_positions
 * sizes (utils.py:463-478), monotone output positions ending at n_elements,
 * n_elements == 2 * packed bytes.  On failure writes a message to msg.
 */
int ecf8_validate_format(const uint8_t *luts, int n_luts, int64_t n_bytes,
                         int64_t packed_bytes, const uint64_t *output_positions,
                         int64_t n_output_positions, int64_t gaps_bytes, int64_t n_elements,
                         int threads_per_block, int bytes_per_thread, char *msg, size_t msg_len);

#ifdef __cplusplus
}
#endif

#endif /* ECF8_H */
