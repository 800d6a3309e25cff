// Host-side part of libecf8: the bitstream encoder (the producer of the
// decoder's input, run offline on the CPU as in the reference), encoder
// output sizing, and the compressed-block format validator.  Declared in
// include/ecf8.h.

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "ecf8.h"

namespace {

// Encoder core shared by sizing and encoding.  The per-symbol bookkeeping
// follows the reference's rule exactly (dfloat/utils.py:387-463): a chunk gap
// is recorded whenever the running bit count enters a chunk with no gap yet
// (total_bits / chunk_bits + 1 > gaps recorded), a format-block position
// whenever it enters a format-block with none yet, and after the last symbol
// the same two checks run once more at the EOF pad position when a partial
// byte remains.  Bits are accumulated 32 at a time and written big-endian.
struct Sink {
  uint8_t *encoded;
  int64_t enc_cap;
  uint8_t *gaps;  // packed nibbles, even chunk high
  int64_t gaps_cap;
  uint64_t *op;
  int64_t op_cap;
  bool write;
  bool overflow = false;
  int64_t n_enc = 0, n_gaps = 0, n_op = 0;

  void put_byte(uint8_t b) {
    if (write) {
      if (n_enc < enc_cap) encoded[n_enc] = b;
      else overflow = true;
    }
    ++n_enc;
  }
  void put_gap(uint32_t gap) {
    if (write) {
      const int64_t byte = n_gaps >> 1;
      if (byte < gaps_cap) {
        if (n_gaps & 1) gaps[byte] = (uint8_t)(gaps[byte] | (gap & 0xF));
        else gaps[byte] = (uint8_t)((gap & 0xF) << 4);
      } else {
        overflow = true;
      }
    }
    ++n_gaps;
  }
  void put_op(uint64_t v) {
    if (write) {
      if (n_op < op_cap) op[n_op] = v;
      else overflow = true;
    }
    ++n_op;
  }
};

int encode_core(const uint8_t *exps, int64_t n, const uint8_t *code_bits, const uint32_t *code_vals,
                int eof_bits, uint32_t eof_value, int bpt, int tpb, Sink &sink) {
  const int64_t chunk_bits = 8LL * bpt;
  const int64_t block_bits = chunk_bits * tpb;
  uint64_t acc = 0;  // pending bits, right-aligned
  int nacc = 0;      // < 32 between symbols
  int64_t total = 0;
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t s = exps[i];
    if (s > 15 || code_bits[s] == 0 || code_bits[s] > 16) return ECF8_ERR_FORMAT;
    if (total / chunk_bits + 1 > sink.n_gaps) sink.put_gap((uint32_t)(total % chunk_bits));
    if (total / block_bits + 1 > sink.n_op) sink.put_op((uint64_t)i);
    const int len = code_bits[s];
    acc = (acc << len) | (code_vals ? (code_vals[s] & ((1u << len) - 1)) : 0u);
    nacc += len;
    total += len;
    if (nacc >= 32) {
      const uint32_t word = (uint32_t)(acc >> (nacc - 32));
      sink.put_byte((uint8_t)(word >> 24));
      sink.put_byte((uint8_t)(word >> 16));
      sink.put_byte((uint8_t)(word >> 8));
      sink.put_byte((uint8_t)word);
      nacc -= 32;
      acc &= (nacc ? ((1ull << nacc) - 1) : 0ull);
    }
  }
  while (nacc >= 8) {
    sink.put_byte((uint8_t)(acc >> (nacc - 8)));
    nacc -= 8;
    acc &= (1ull << nacc) - 1;
  }
  if (nacc > 0) {  // final partial byte, padded with the EOF code's leading bits
    if (total / chunk_bits + 1 > sink.n_gaps) sink.put_gap((uint32_t)(total % chunk_bits));
    if (total / block_bits + 1 > sink.n_op) sink.put_op((uint64_t)n);
    if (eof_bits < 1 || eof_bits > 24) return ECF8_ERR_FORMAT;
    const uint64_t v = (acc << eof_bits) | (eof_value & ((1u << eof_bits) - 1));
    const int size = nacc + eof_bits;
    sink.put_byte((uint8_t)(size >= 8 ? v >> (size - 8) : v << (8 - size)));
  }
  sink.put_op((uint64_t)n);
  const int64_t fb_bytes = (int64_t)bpt * tpb;
  const int64_t n_fb = (sink.n_enc + fb_bytes - 1) / fb_bytes;
  while (sink.n_gaps < n_fb * tpb) sink.put_gap(0);
  return sink.overflow ? ECF8_ERR_CAPACITY : ECF8_OK;
}

bool geometry_ok(int bpt, int tpb) {
  return bpt >= 2 && bpt <= 64 && tpb >= 2 && tpb <= 4096 && (tpb % 2) == 0;
}

}  // namespace

extern "C" const char *ecf8_version(void) { return "ecf8_amd 0.1.0 (gfx950)"; }

extern "C" const char *ecf8_status_string(int status) {
  switch (status) {
    case ECF8_OK: return "ok";
    case ECF8_ERR_INVALID_ARG: return "invalid argument";
    case ECF8_ERR_UNSUPPORTED: return "unsupported format geometry";
    case ECF8_ERR_MISALIGNED: return "misaligned device buffer";
    case ECF8_ERR_FORMAT: return "malformed compressed block";
    case ECF8_ERR_HIP: return "HIP runtime error";
    case ECF8_ERR_CAPACITY: return "output buffer too small";
    default: return "unknown status";
  }
}

extern "C" int ecf8_encoded_sizes(const uint8_t *exponents, int64_t n, const uint8_t *code_bits,
                                  int bytes_per_thread, int threads_per_block, int64_t *n_bytes,
                                  int64_t *gaps_bytes, int64_t *n_output_positions) {
  if ((n > 0 && !exponents) || !code_bits || n < 0 || !n_bytes || !gaps_bytes ||
      !n_output_positions)
    return ECF8_ERR_INVALID_ARG;
  if (!geometry_ok(bytes_per_thread, threads_per_block)) return ECF8_ERR_UNSUPPORTED;
  Sink sink{nullptr, 0, nullptr, 0, nullptr, 0, false};
  // the EOF code only affects the pad byte's value, not the sizes
  const int rc = encode_core(exponents, n, code_bits, nullptr, 1, 0, bytes_per_thread,
                             threads_per_block, sink);
  if (rc != ECF8_OK) return rc;
  *n_bytes = sink.n_enc;
  *gaps_bytes = (sink.n_gaps + 1) / 2;
  *n_output_positions = sink.n_op;
  return ECF8_OK;
}

extern "C" int ecf8_encode_exponents(const uint8_t *exponents, int64_t n, const uint8_t *code_bits,
                                     const uint32_t *code_vals, int eof_bits, uint32_t eof_value,
                                     int bytes_per_thread, int threads_per_block, uint8_t *encoded,
                                     int64_t encoded_capacity, uint8_t *gaps, int64_t gaps_capacity,
                                     uint64_t *output_positions,
                                     int64_t output_positions_capacity) {
  if ((n > 0 && !exponents) || !code_bits || !code_vals || n < 0 || !output_positions ||
      (encoded_capacity > 0 && !encoded) || (gaps_capacity > 0 && !gaps))
    return ECF8_ERR_INVALID_ARG;
  if (!geometry_ok(bytes_per_thread, threads_per_block)) return ECF8_ERR_UNSUPPORTED;
  Sink sink{encoded, encoded_capacity, gaps, gaps_capacity, output_positions,
            output_positions_capacity, true};
  return encode_core(exponents, n, code_bits, code_vals, eof_bits, eof_value, bytes_per_thread,
                     threads_per_block, sink);
}

extern "C" int ecf8_validate_format(const uint8_t *luts, int n_luts, int64_t n_bytes,
                                    int64_t packed_bytes, const uint64_t *output_positions,
                                    int64_t n_output_positions, int64_t gaps_bytes,
                                    int64_t n_elements, int threads_per_block,
                                    int bytes_per_thread, char *msg, size_t msg_len) {
  auto fail = [&](int rc, const char *fmt, long long a, long long b) {
    if (msg && msg_len) snprintf(msg, msg_len, fmt, a, b);
    return rc;
  };
  if (!luts || !output_positions)
    return fail(ECF8_ERR_INVALID_ARG, "null luts (%lld) or output_positions (%lld)", !luts,
                !output_positions);
  if (!geometry_ok(bytes_per_thread, threads_per_block))
    return fail(ECF8_ERR_UNSUPPORTED, "geometry %lld x %lld unsupported", bytes_per_thread,
                threads_per_block);
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS)
    return fail(ECF8_ERR_FORMAT, "n_luts=%lld outside [2, %lld]", n_luts, ECF8_MAX_LUTS);
  if (n_elements != 2 * packed_bytes)
    return fail(ECF8_ERR_FORMAT, "n_elements=%lld != 2 * packed bytes %lld", n_elements,
                packed_bytes);
  const uint8_t *lens = luts + 256 * (n_luts - 1);
  // first-level and second-level entries: a symbol with a code length, or
  // (first level only) a pointer to an existing second-level row
  for (int r = 0; r < n_luts - 1; ++r) {
    for (int k = 0; k < 256; ++k) {
      const int v = luts[256 * r + k];
      if (v >= 240) {
        if (r != 0) return fail(ECF8_ERR_FORMAT, "pointer in second-level row %lld at %lld", r, k);
        const int row = 256 - v;
        if (row > n_luts - 2)
          return fail(ECF8_ERR_FORMAT, "pointer to row %lld of %lld rows", row, n_luts - 2);
      } else if (v > 15) {
        return fail(ECF8_ERR_FORMAT, "entry %lld is not an exponent (row %lld)", v, r);
      }
    }
  }
  // Entries of symbols without a code (length 0) are legal: the builder's
  // forward fill starts from 0 (utils.py:352), so keys before the first code
  // in a row read as symbol 0, reachable only through the EOF code's bits.
  for (int v = 0; v < 16; ++v)
    if (lens[v] > 16) return fail(ECF8_ERR_FORMAT, "symbol %lld has code length %lld", v, lens[v]);
  const int64_t fb_bytes = (int64_t)bytes_per_thread * threads_per_block;
  const int64_t n_fb = (n_bytes + fb_bytes - 1) / fb_bytes;
  if (n_output_positions != n_fb + 1)
    return fail(ECF8_ERR_FORMAT, "%lld output positions for %lld format-blocks", n_output_positions,
                n_fb);
  if (gaps_bytes != n_fb * threads_per_block / 2)
    return fail(ECF8_ERR_FORMAT, "%lld gap bytes for %lld format-blocks", gaps_bytes, n_fb);
  if (output_positions[0] != 0 && n_fb > 0)
    return fail(ECF8_ERR_FORMAT, "output_positions[0]=%lld, expected %lld",
                (long long)output_positions[0], 0);
  for (int64_t b = 0; b < n_fb; ++b)
    if (output_positions[b + 1] < output_positions[b])
      return fail(ECF8_ERR_FORMAT, "output_positions decrease at %lld (%lld)", b,
                  (long long)output_positions[b + 1]);
  if ((int64_t)output_positions[n_fb] != n_elements)
    return fail(ECF8_ERR_FORMAT, "last output position %lld != n_elements %lld",
                (long long)output_positions[n_fb], n_elements);
  const int64_t max_syms = (int64_t)threads_per_block * 8 * bytes_per_thread;
  for (int64_t b = 0; b < n_fb; ++b)
    if ((int64_t)(output_positions[b + 1] - output_positions[b]) > max_syms)
      return fail(ECF8_ERR_FORMAT, "format-block %lld holds more than %lld symbols", b, max_syms);
  return ECF8_OK;
}
