// Host codec under AddressSanitizer / UndefinedBehaviorSanitizer: the
// validator, both table builders' host path, the code recovery and the two
// encoders of libecf8 are fed real compressed blocks (written by the test
// that builds this file) and then corrupted LUTs, positions, sizes and code
// tables.  Every buffer is heap-allocated at exactly the size the call is
// told, so a read or write past it is reported by the sanitizer.  The
// harness checks statuses only where they are determined (the original
// block must validate and re-encode byte for byte); on corrupt input any
// status is acceptable, a memory error or undefined behaviour is not.
//
// Input file: repeated records of
//   i32 n_luts, i64 n_bytes, i64 n_elements, i64 n_op, i64 gaps_bytes,
//   i32 rows, i32 cols (the block as a [rows, cols] weight, rows % 16 == 0,
//   cols % 128 == 0), then luts, encoded, packed nibbles, op (u64),
//   gaps, the exponents (n_elements bytes), the e4m3fn weight bytes.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <memory>
#include <vector>

#include "ecf8.h"
#include "ecf8_tile.h"

namespace {

struct Block {
  int n_luts = 0, rows = 0, cols = 0;
  int64_t n_bytes = 0, n_elements = 0, n_op = 0, gaps_bytes = 0;
  std::vector<uint8_t> luts, encoded, packed, gaps, exps, weight;
  std::vector<uint64_t> op;
};

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t rnd() {
  g_state ^= g_state << 13;
  g_state ^= g_state >> 7;
  g_state ^= g_state << 17;
  return g_state;
}
int rnd_int(int lo, int hi) { return lo + (int)(rnd() % (uint64_t)(hi - lo + 1)); }

// A heap copy of exactly n bytes (n may be 0: a 1-byte allocation nobody reads).
template <class T>
std::unique_ptr<T[]> exact(const T *src, size_t n) {
  std::unique_ptr<T[]> p(new T[n ? n : 1]);
  if (n) memcpy(p.get(), src, n * sizeof(T));
  return p;
}

bool read_block(FILE *f, Block &b) {
  int32_t i32[1];
  int64_t i64[4];
  int32_t rc[2];
  if (fread(i32, 4, 1, f) != 1) return false;
  if (fread(i64, 8, 4, f) != 4 || fread(rc, 4, 2, f) != 2) return false;
  b.n_luts = i32[0];
  b.n_bytes = i64[0];
  b.n_elements = i64[1];
  b.n_op = i64[2];
  b.gaps_bytes = i64[3];
  b.rows = rc[0];
  b.cols = rc[1];
  auto rd = [&](auto &v, size_t n) {
    v.resize(n);
    return fread(v.data(), sizeof(v[0]), n, f) == n;
  };
  return rd(b.luts, (size_t)b.n_luts * 256) && rd(b.encoded, (size_t)b.n_bytes) &&
         rd(b.packed, (size_t)b.n_elements / 2) && rd(b.op, (size_t)b.n_op) &&
         rd(b.gaps, (size_t)b.gaps_bytes) && rd(b.exps, (size_t)b.n_elements) &&
         rd(b.weight, (size_t)b.n_elements);
}

int validate(const uint8_t *luts, int n_luts, int64_t n_bytes, int64_t packed,
             const uint64_t *op, int64_t n_op, int64_t gaps_bytes, int64_t n_elements) {
  char msg[160];
  return ecf8_validate_format(luts, n_luts, n_bytes, packed, op, n_op, gaps_bytes, n_elements,
                              512, 8, msg, sizeof msg);
}

// Every host entry point that takes a LUT stack, on this one.
void luts_calls(const uint8_t *luts_src, int n_luts, const Block &b) {
  const size_t nl = n_luts > 0 ? (size_t)n_luts * 256 : 0;
  auto luts = exact(luts_src, nl);
  validate(luts.get(), n_luts, b.n_bytes, b.n_elements / 2, b.op.data(), b.n_op, b.gaps_bytes,
           b.n_elements);
  for (int kind : {ECF8_TABLE_ANY, ECF8_TABLE_MULTI, ECF8_TABLE_DFA}) {
    std::unique_ptr<uint32_t[]> table(new uint32_t[ECF8_TABLE_BYTES / 4]);
    int got = -1;
    ecf8_build_table_host(luts.get(), n_luts, kind, table.get(), &got);
  }
  uint8_t bits[16];
  uint32_t vals[16];
  if (ecf8_code_from_luts(luts.get(), n_luts, bits, vals) != ECF8_OK) return;
  int64_t nbytes = 0, nseg = 0;
  auto w = exact(b.weight.data(), b.weight.size());
  if (ecf8_tile_sizes(w.get(), b.rows, b.cols, bits, &nbytes, &nseg) != ECF8_OK) return;
  auto stream = std::unique_ptr<uint8_t[]>(new uint8_t[nbytes ? nbytes : 1]);
  std::unique_ptr<uint32_t[]> seg_off(new uint32_t[nseg + 1]), gaps(new uint32_t[8 * nseg]);
  std::unique_ptr<uint8_t[]> other(new uint8_t[1024 * nseg]);
  ecf8_tile_encode(w.get(), b.rows, b.cols, bits, vals, stream.get(), nbytes, seg_off.get(),
                   gaps.get(), other.get(), 2);
}

// The bitstream encoder under a code table and exponent array.
int encode(const uint8_t *exps_src, int64_t n, const uint8_t *bits, const uint32_t *vals,
           int eof_bits, uint32_t eof_val, int64_t shrink, std::vector<uint8_t> *out_enc) {
  auto exps = exact(exps_src, (size_t)n);
  int64_t nb = 0, gb = 0, no = 0;
  int rc = ecf8_encoded_sizes(exps.get(), n, bits, 8, 512, &nb, &gb, &no);
  if (rc != ECF8_OK) return rc;
  const int64_t cap = nb > shrink ? nb - shrink : 0;
  std::unique_ptr<uint8_t[]> enc(new uint8_t[cap ? cap : 1]), gaps(new uint8_t[gb ? gb : 1]);
  std::unique_ptr<uint64_t[]> op(new uint64_t[no ? no : 1]);
  rc = ecf8_encode_exponents(exps.get(), n, bits, vals, eof_bits, eof_val, 8, 512, enc.get(), cap,
                             gaps.get(), gb, op.get(), no);
  if (rc == ECF8_OK && out_enc) out_enc->assign(enc.get(), enc.get() + cap);
  return rc;
}

int check_block(const Block &b) {
  int failures = 0;
  if (validate(b.luts.data(), b.n_luts, b.n_bytes, b.n_elements / 2, b.op.data(), b.n_op,
               b.gaps_bytes, b.n_elements) != ECF8_OK) {
    fprintf(stderr, "original block does not validate\n");
    ++failures;
  }
  uint8_t bits[16];
  uint32_t vals[16];
  if (ecf8_code_from_luts(b.luts.data(), b.n_luts, bits, vals) != ECF8_OK) {
    fprintf(stderr, "original block's code not recovered\n");
    return failures + 1;
  }
  // the EOF code: the LUT builder's length row has no EOF entry, so take the
  // encoder's padding from the recovered code's unused prefix
  luts_calls(b.luts.data(), b.n_luts, b);

  for (int it = 0; it < 150; ++it) {
    // corrupt LUT bytes and row counts
    std::vector<uint8_t> luts = b.luts;
    const int flips = rnd_int(1, 8);
    for (int f = 0; f < flips; ++f) {
      const size_t at = rnd() % luts.size();
      luts[at] = (rnd() & 1) ? (uint8_t)rnd() : (uint8_t)(240 + rnd_int(0, 15));
    }
    int n_luts = b.n_luts;
    if (rnd() % 4 == 0) n_luts = rnd_int(0, (int)(luts.size() / 256));
    luts_calls(luts.data(), n_luts, b);

    // corrupt output positions and sizes
    std::vector<uint64_t> op = b.op;
    const int hits = rnd_int(1, 4);
    for (int h = 0; h < hits; ++h) {
      const size_t at = rnd() % op.size();
      switch (rnd() % 4) {
        case 0: op[at] = rnd(); break;
        case 1: op[at] = op[at] ? op[at] - 1 : 1; break;
        case 2: op[at] += (uint64_t)rnd_int(1, 100000); break;
        default: op[at] = (uint64_t)b.n_elements * 2; break;
      }
    }
    auto opx = exact(op.data(), op.size());
    const int64_t n_op = rnd() % 5 == 0 ? (int64_t)op.size() - rnd_int(0, 1) : (int64_t)op.size();
    validate(b.luts.data(), b.n_luts, b.n_bytes + rnd_int(-64, 64), b.n_elements / 2, opx.get(),
             n_op, b.gaps_bytes + rnd_int(-8, 8), b.n_elements + 2 * rnd_int(-3, 3));

    // the encoder with corrupt code tables, exponents and short capacities
    uint8_t cb[16];
    uint32_t cv[16];
    memcpy(cb, bits, 16);
    memcpy(cv, vals, 16);
    if (rnd() & 1) cb[rnd() % 16] = (uint8_t)rnd_int(0, 24);
    if (rnd() & 1) cv[rnd() % 16] = (uint32_t)rnd();
    const int64_t n = 2 * rnd_int(1, 4096);
    std::vector<uint8_t> ex(b.exps.begin(), b.exps.begin() + n);
    if (rnd() & 1) ex[rnd() % n] = (uint8_t)rnd();
    encode(ex.data(), n, cb, cv, rnd_int(0, 20), (uint32_t)rnd(), rnd_int(0, 3), nullptr);
  }
  return failures;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s blocks.bin\n", argv[0]);
    return 2;
  }
  FILE *f = fopen(argv[1], "rb");
  if (!f) return 2;
  int failures = 0, blocks = 0;
  Block b;
  while (read_block(f, b)) {
    failures += check_block(b);
    ++blocks;
  }
  fclose(f);
  printf("blocks %d failures %d\n", blocks, failures);
  return failures ? 1 : 0;
}
