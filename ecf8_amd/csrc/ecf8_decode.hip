// ECF8 decode engine for MI355X (gfx950): device kernels and their C-ABI
// launchers (declared in include/ecf8.h).
//
// Format (the reference's on-disk contract, dfloat/utils.py:207-499):
//   * exponents e_i = (b_i >> 3) & 0xF are Huffman-coded MSB-first into
//     `encoded`; sign+mantissa nibbles o_i are packed two per byte, even
//     element in the high nibble (`packed_other_4bits`);
//   * chunk g = bits [64g, 64g+64) of `encoded`; its 4-bit gap is the offset
//     of the first code that starts inside it; chunk g owns every code whose
//     start lies in [64g + gap_g, 64g + 64) (dfloat/run/decode.cu:85-112);
//   * a format-block is `threads_per_block` consecutive chunks; its first
//     owned symbol is element output_positions[b] (utils.py:405-406).
// Decode rule per symbol (decode.cu:86-91): with W the next 16 bits,
// v = L0[W >> 8]; if v >= 240 then v = L[256 - v][W & 0xFF]; length =
// Llen[v]; the output byte is (o & 8) << 4 | v << 3 | (o & 7).
//
// MI355X design: a persistent grid, one workgroup per format-block at a
// time and one chunk per lane; the next block's bitstream and positions are
// fetched a whole block ahead.  Per block:
//   1. each lane decodes the codes its chunk owns through a table derived
//      once per compressed block (ecf8_tables.cpp), held in LDS:
//        DFA   kernel: a byte automaton, exactly 8 lookups per chunk plus
//              one (rarely two) for the code in flight at the chunk's end;
//              no data-dependent loop, the entries stay in registers;
//        MULTI kernel: 12-bit windows, up to 4 symbols per lookup, a
//              predicated loop, exponents ORed into a lane-private LDS run
//              (any LUT stack, e.g. one with a 1-bit code);
//   2. the per-chunk symbol counts are prefix-summed (wave64 DPP scan +
//      per-wave totals in LDS), giving each lane its output offset;
//   3. each lane ORs its exponent nibbles into a dense LDS staging buffer at
//      that offset (double-buffered across blocks, sized from the largest
//      block of the tensor like the reference's shared_mem_size);
//   4. the staging buffer is swept in 16-element segments: 8 exponent
//      nibbles + 8 bytes of sign/mantissa nibbles (prefetched at block
//      start) become 16 FP8 bytes with bitfield inserts and byte permutes,
//      stored as one 128-bit store (byte stores only on the two partial
//      segments at the block edges).
// All work is integer VALU/LDS; the HBM traffic is the compressed bytes read
// once and the FP8 bytes written once.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <vector>

#include "ecf8.h"
#include "ecf8_dev.h"
#include "ecf8_layout.h"

namespace {

using namespace ecf8;
using namespace ecf8::dev;

// Sum of the totals of the waves before this one (s_wave_sum[w] = total of
// wave w): lanes 0..kWaves-1 load one total each, a DPP prefix inside the
// first row adds them up, and this wave's entry is read back.
// Optionally also the total over all waves.
template <int kWaves>
__device__ __forceinline__ int waves_before(const int *s_wave_sum, int lane, int wave,
                                            int *total = nullptr) {
  const int own = lane < kWaves ? s_wave_sum[lane] : 0;
  int t = own;
  if (kWaves > 1) t += __builtin_amdgcn_update_dpp(0, t, 0x111, 0xF, 0xF, true);  // row_shr:1
  if (kWaves > 2) t += __builtin_amdgcn_update_dpp(0, t, 0x112, 0xF, 0xF, true);  // row_shr:2
  if (kWaves > 4) t += __builtin_amdgcn_update_dpp(0, t, 0x114, 0xF, 0xF, true);  // row_shr:4
  if (kWaves > 8) t += __builtin_amdgcn_update_dpp(0, t, 0x118, 0xF, 0xF, true);  // row_shr:8
  if (total) *total = __builtin_amdgcn_readlane(t, kWaves - 1);
  return __builtin_amdgcn_readlane(t - own, __builtin_amdgcn_readfirstlane(wave));
}

typedef uint32_t u32x3_a8 __attribute__((ext_vector_type(3), aligned(8)));

// A chunk as fetched: 12 raw bytes from the chunk start (8 chunk bytes, 2
// look-ahead bytes, 2 unused; little-endian dwords) and the byte holding its
// gap nibble.  Fetching never waits; the bytes are interpreted a whole
// decode phase later.
struct RawChunk {
  u32x3_a8 v;
  uint32_t gap_byte;
};

// Unconditional 96-bit load of chunk g, the address clamped to the last
// full 12-byte window so it stays in bounds; lanes near the stream end are
// re-read byte-wise when the chunk is finished.
__device__ __forceinline__ RawChunk fetch_chunk(const uint8_t *__restrict__ encoded, uint32_t last12,
                                                const uint8_t *__restrict__ gaps, uint32_t g) {
  RawChunk r;
  const uint32_t b = g * kChunkBytes;
  r.v = *reinterpret_cast<const u32x3_a8 *>(encoded + (b < last12 ? b : last12));
  r.gap_byte = gaps[g >> 1];
  return r;
}

__device__ __forceinline__ uint32_t gap_of(uint32_t gap_byte, uint32_t g) {
  return (g & 1) ? (gap_byte & 0xFu) : (gap_byte >> 4);
}

// The chunk's 10 bytes as little-endian dwords (byte k of the chunk in bits
// 8(k%4).. of dword k/4), bytes past n_bytes read as zero.
__device__ __forceinline__ uint3 chunk_bytes(const RawChunk &r, const uint8_t *__restrict__ encoded,
                                             uint32_t n_bytes, uint32_t g, bool vector_ok) {
  const uint32_t b = g * kChunkBytes;
  if (vector_ok && b + 12 <= n_bytes) return make_uint3(r.v.x, r.v.y, r.v.z);
  uint32_t d[3] = {0u, 0u, 0u};
  for (int i = 0; i < kChunkBytes + 2; ++i) {
    const uint32_t j = b + i;
    d[i >> 2] |= (j < n_bytes ? (uint32_t)encoded[j] : 0u) << (8 * (i & 3));
  }
  return make_uint3(d[0], d[1], d[2]);
}

// The 8 sign/mantissa bytes of the 16 outputs at the 16-aligned gpos, read
// byte-wise with bounds checks.
__device__ __forceinline__ uint2 load_nibbles_checked(const uint8_t *__restrict__ packed,
                                                      uint32_t n_elements, uint32_t gpos) {
  uint32_t t[2] = {0u, 0u};
  for (int i = 0; i < 8; ++i) {
    const uint32_t q = (gpos >> 1) + i;
    const uint32_t b = q < (n_elements >> 1) ? packed[q] : 0u;
    t[i >> 2] |= b << (8 * (i & 3));
  }
  return make_uint2(t[0], t[1]);
}

// Dwords of one staging buffer holding `cap` symbols from a 16-aligned base
// (<= 15 leading nibbles), rounded to 16 bytes.
__host__ __device__ constexpr int stage_dwords(int cap) {
  return ((((cap + 30) >> 4) * 2) + 3) & ~3;
}

// A format-block's output range and its staging geometry (wave-uniform).
struct BlockRange {
  uint32_t start, end;  // outputs [start, end) are written
  uint32_t base;        // 16-element aligned sweep origin
  int lead;             // start - base
  int seg_dw;           // staging dwords in use (whole 16-element segments)
  int nseg;             // 16-element segments to sweep
};

__device__ __forceinline__ BlockRange block_range(uint32_t op_lo, uint32_t op_hi,
                                                  uint32_t n_elements, int stage_cap) {
  BlockRange r;
  r.start = op_lo;
  const uint32_t end = op_hi < n_elements ? op_hi : n_elements;
  int total = (int)end - (int)op_lo;
  if (total < 0 || op_lo > n_elements) total = 0;  // malformed positions write nothing
  if (total > stage_cap) total = stage_cap;         // an understated largest block
  r.end = op_lo + (uint32_t)total;
  r.base = op_lo & ~15u;
  r.lead = (int)(op_lo - r.base);
  const int stage_nib = total > 0 ? r.lead + total : 0;
  r.seg_dw = ((stage_nib + 15) >> 4) * 2;
  r.nseg = r.seg_dw >> 1;
  return r;
}

// Sign/mantissa bytes of this lane's first two segments, loaded at block
// start so they arrive during the decode (a first segment past nseg
// re-reads the last one; a second one is not loaded).
__device__ __forceinline__ void prefetch_nibbles(const BlockRange &br, const uint8_t *packed,
                                                 uint32_t last8, int tid, int threads, uint2 &pre0,
                                                 uint2 &pre1) {
  const int last_seg = br.nseg > 0 ? br.nseg - 1 : 0;
  const uint32_t q0 = (br.base >> 1) + 8u * (uint32_t)min(tid, last_seg);
  const uint32_t q1 = (br.base >> 1) + 8u * (uint32_t)min(tid + threads, last_seg);
  // non-temporal: each nibble byte is read exactly once (measured on
  // MI355X: 74.0 -> 72.1 us per Qwen3-8B layer).  The chunk loads stay
  // ordinary: neighbouring lanes' 12-byte windows share cache lines.
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 a0 = __builtin_nontemporal_load(
      reinterpret_cast<const u32x2 *>(packed + (q0 < last8 ? q0 : last8)));
  // only lanes with a second segment load it: under the non-temporal hint
  // a repeated address is fetched again rather than served from cache
  // (74 -> 72 us per Qwen3-8B layer when the lanes past nseg stopped
  // re-reading the last segment)
  u32x2 a1 = {0u, 0u};
  if (tid + threads < br.nseg)
    a1 = __builtin_nontemporal_load(
        reinterpret_cast<const u32x2 *>(packed + (q1 < last8 ? q1 : last8)));
  pre0 = make_uint2(a0.x, a0.y);
  pre1 = make_uint2(a1.x, a1.y);
}

// LDS slots for the two edge segments of a block (first and last, which it
// shares with its neighbours): 16 merged bytes, then gpos, start, end.
constexpr int kEdgeSlotDwords = 8;
constexpr int kEdgeDwords = 2 * kEdgeSlotDwords;

// Step 4: merge the staged exponents with the sign/mantissa nibbles and
// store the block's FP8 bytes: whole segments as one 128-bit store each;
// the edge segments are parked in s_edge and stored byte-wise by
// flush_edges after the next barrier, spread over lanes.
template <int kThreads, bool kChecked>
__device__ __forceinline__ void write_block(const uint32_t *stage, const BlockRange &br,
                                            uint2 pre0, uint2 pre1,
                                            const uint8_t *__restrict__ packed,
                                            uint32_t n_elements, uint8_t *__restrict__ out,
                                            uint32_t *s_edge, int tid) {
  for (int s = tid, k = 0; s < br.nseg; s += kThreads, ++k) {
    const uint2 ev = reinterpret_cast<const uint2 *>(stage)[s];
    const uint32_t gpos = br.base + 16u * (uint32_t)s;
    uint2 ov = k == 0 ? pre0 : pre1;
    if (kChecked || k > 1 || gpos + 16 > n_elements)
      ov = load_nibbles_checked(packed, n_elements, gpos);
    const uint2 lo = merge8(ev.x, ov.x);
    const uint2 hi8 = merge8(ev.y, ov.y);
    if (gpos >= br.start && gpos + 16 <= br.end) {
      // streaming (non-temporal) store: the output is written once and read
      // by the next kernel from HBM, so it should not displace cached input
      const u32x4 w = {lo.x, lo.y, hi8.x, hi8.y};
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(out + gpos));
    } else {  // only the first and the last segment can be partial
      uint32_t *const e = s_edge + (s == 0 ? 0 : kEdgeSlotDwords);
      *reinterpret_cast<uint4 *>(e) = make_uint4(lo.x, lo.y, hi8.x, hi8.y);
      e[4] = gpos;
      e[5] = br.start;
      e[6] = br.end;
    }
  }
}

// Store the in-range bytes of the edge segments parked by the last
// write_block (lanes first..first+31 of the workgroup, one byte each), then
// mark the slots empty.  Called between a barrier that follows that
// write_block and the barrier before the next one.  The callers pass the
// last wave, which has the fewest segments to write, so the extra LDS round
// trip lands on the wave with the most slack before the next barrier.
__device__ __forceinline__ void flush_edges(uint32_t *s_edge, uint8_t *__restrict__ out,
                                            int tid, int first) {
  const int t = tid - first;
  if ((unsigned)t < 32u) {
    uint32_t *const e = s_edge + (t >> 4) * kEdgeSlotDwords;
    const uint32_t i = (uint32_t)t & 15u;
    const uint4 meta = *reinterpret_cast<const uint4 *>(e + 4);  // gpos, start, end
    uint32_t w = e[i >> 2];
    asm volatile("" : "+v"(w));  // both reads before the range test: one LDS round trip
    const uint32_t q = meta.x + i;
    const uint32_t b = (w >> (8 * (i & 3))) & 0xFFu;
    const bool in_range = q >= meta.y && q < meta.z;
    if (in_range) out[q] = (uint8_t)b;
    if (i == 0) {
      e[5] = 0u;
      e[6] = 0u;
    }
  }
}

// ---------------------------------------------------------------------------
// Scaled bf16 output (ecf8_decode_bf16)
// ---------------------------------------------------------------------------

// One Linear of the block: elements [start, start + rows * cols) are its
// row-major weight.  The row of element q is (q - start) / cols, computed as
// umulhi(q - start, magic) >> shift (exact for q - start < 2^31: magic =
// ceil(2^(31 + s) / cols), shift = s - 1, s = ceil(log2 cols)).
struct ScalePart {
  uint32_t start, cols, magic, shift;
  const float *scale;  // [rows / 128][cols / 128]
};
struct ScaleParts {
  ScalePart p[ECF8_MAX_SCALED_PARTS];
  int n;
};

// The part holding element q.
__device__ __forceinline__ int part_of(const ScalePart *s_parts, int n_parts, uint32_t q) {
  int k = 0;
  for (int j = 1; j < n_parts; ++j) k += q >= s_parts[j].start ? 1 : 0;
  return k;
}

// Block scale of the 8-element half-segment at gpos (gpos < n_elements; it
// never straddles a row or a part: both are multiples of 16), searching
// forward from part k0, which starts at or before gpos (the block's first
// part: a block rarely spans two).
__device__ __forceinline__ float segment_scale(const ScalePart *s_parts, int n_parts, int k0,
                                               uint32_t gpos) {
  int k = k0;
  while (k + 1 < n_parts && gpos >= s_parts[k + 1].start) ++k;
  const uint32_t idx = gpos - s_parts[k].start;
  const uint32_t cols = s_parts[k].cols;
  const uint32_t row = __umulhi(idx, s_parts[k].magic) >> s_parts[k].shift;
  const uint32_t col = idx - row * cols;
  return as_global(s_parts[k].scale)[(row >> 7) * (cols >> 7) + (col >> 7)];
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Four FP8 bytes (element order) -> four bf16 of fp8 x sc: exact FP8 -> f32
// conversions, one f32 product each, round to nearest even to bf16.
__device__ __forceinline__ uint2 fp8x4_scaled_bf16(uint32_t w, float sc) {
  const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false) * sc;
  const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true) * sc;
  return make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(a, bf16x2)),
                    __builtin_bit_cast(uint32_t, __builtin_convertvector(b, bf16x2)));
}

// Scaled bf16 output is written in half-segments of 8 elements: staging
// dword h (8 exponent nibbles) and the nibble dword of the same elements
// make 8 FP8 bytes, converted to 16 bytes of bf16 and stored by one lane.
// Lane t takes half-segments t, t + threads, ..., so each store
// instruction writes 64 x 16 contiguous bytes.  With whole 16-element
// segments per lane, each store covers every other 16 bytes of twice the
// span.  Measured on MI355X per FLUX double block (226.5 M elements):
// 138.9 us with whole segments, 131.6 us with half-segments.
// Half-segments per lane whose nibbles load at block start, and of those,
// the ones whose scale loads before the staging ORs (the rest look theirs up
// in the store phase).  All four prefetched, FLUX double block: 127.3 us
// against 130.6 with two (3 rotated sets), 0.1409 against 0.1415 ms on the
// bench line (10 sets, four rounds each).
constexpr int kHalfPrefetch = 4;
constexpr int kScalePrefetch = 4;

// Sign/mantissa dwords of this lane's first kHalfPrefetch half-segments,
// loaded at block start (non-temporal; only lanes that have the
// half-segment load it, the first one clamped to the block's last).
__device__ __forceinline__ void prefetch_nibbles_half(const BlockRange &br,
                                                      const uint8_t *__restrict__ packed,
                                                      uint32_t last4, int tid, int threads,
                                                      uint32_t (&pre)[kHalfPrefetch]) {
  const int nh = 2 * br.nseg;
#pragma unroll
  for (int k = 0; k < kHalfPrefetch; ++k) {
    const int h = tid + k * threads;
    const int hc = k == 0 ? min(h, nh > 0 ? nh - 1 : 0) : h;
    const uint32_t q = (br.base >> 1) + 4u * (uint32_t)hc;
    pre[k] = 0u;
    if (k == 0 || h < nh)
      pre[k] = __builtin_nontemporal_load(
          reinterpret_cast<const uint32_t *>(packed + (q < last4 ? q : last4)));
  }
}

// write_block for scaled bf16 output (n_elements a multiple of 16).  The
// half-segments holding the block's first and last output, when partial,
// are parked in the edge slots (8 merged bytes, then gpos, start, end and
// the scale) for flush_edges_bf16.
template <int kThreads>
__device__ __forceinline__ void write_block_bf16(const uint32_t *stage, const BlockRange &br,
                                                 const uint32_t (&pre)[kHalfPrefetch],
                                                 const float (&sc)[kScalePrefetch],
                                                 const uint8_t *__restrict__ packed,
                                                 uint32_t n_elements, uint16_t *__restrict__ out16,
                                                 uint32_t *s_edge, int tid,
                                                 const ScalePart *s_parts, int n_parts, int k0) {
  const int nh = 2 * br.nseg;
  auto half = [&](int h, uint32_t ov, float s) {
    const uint32_t gpos = br.base + 8u * (uint32_t)h;
    const uint2 f = merge8(stage[h], ov);
    if (gpos >= br.start && gpos + 8 <= br.end) {
      const uint2 b0 = fp8x4_scaled_bf16(f.x, s), b1 = fp8x4_scaled_bf16(f.y, s);
      __builtin_nontemporal_store(u32x4{b0.x, b0.y, b1.x, b1.y},
                                  reinterpret_cast<u32x4 *>(out16 + gpos));
    } else if (gpos + 8 > br.start && gpos < br.end) {  // holds the first or last output
      uint32_t *const e = s_edge + (gpos <= br.start ? 0 : kEdgeSlotDwords);
      e[0] = f.x;
      e[1] = f.y;
      e[4] = gpos;
      e[5] = br.start;
      e[6] = br.end;
      e[7] = __float_as_uint(s);
    }
  };
  // positions clamped into the tensor for the lookups and loads of
  // half-segments past the block's outputs (their results are discarded)
  auto at = [&](int h) { return min(br.base + 8u * (uint32_t)h, n_elements - 8u); };
#pragma unroll
  for (int k = 0; k < kHalfPrefetch; ++k) {
    const int h = tid + k * kThreads;
    if (h < nh) {
      // k is a constant after unrolling: the first kScalePrefetch scales
      // were loaded before the ORs, the others are looked up here
      const float s = k < kScalePrefetch ? sc[k < kScalePrefetch ? k : 0]
                                         : segment_scale(s_parts, n_parts, k0, at(h));
      half(h, pre[k], s);
    }
  }
  // rarely any: blocks of more than kHalfPrefetch * kThreads half-segments
  for (int h = tid + kHalfPrefetch * kThreads; h < nh; h += kThreads)
    half(h, *reinterpret_cast<const uint32_t *>(packed + (at(h) >> 1)),
         segment_scale(s_parts, n_parts, k0, at(h)));
}

// flush_edges for scaled bf16 output: 8 elements per slot, one per lane,
// 16-bit stores.
__device__ __forceinline__ void flush_edges_bf16(uint32_t *s_edge, uint16_t *__restrict__ out16,
                                                 int tid, int first) {
  const int t = tid - first;
  if ((unsigned)t < 16u) {
    uint32_t *const e = s_edge + (t >> 3) * kEdgeSlotDwords;
    const uint32_t i = (uint32_t)t & 7u;
    const uint4 meta = *reinterpret_cast<const uint4 *>(e + 4);  // gpos, start, end, scale
    uint32_t w = e[i >> 2];
    asm volatile("" : "+v"(w));  // both reads before the range test: one LDS round trip
    const uint32_t q = meta.x + i;
    const uint32_t b = (w >> (8 * (i & 3))) & 0xFFu;
    const f32x2 v = f32x2{__builtin_amdgcn_cvt_f32_fp8((int)b, 0), 0.f} * __uint_as_float(meta.w);
    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    const bool in_range = q >= meta.y && q < meta.z;
    if (in_range) out16[q] = (uint16_t)(hb & 0xFFFFu);
    if (i == 0) {
      e[5] = 0u;
      e[6] = 0u;
    }
  }
}

// ===========================================================================
// DFA kernel (tables of kind ECF8_TABLE_DFA)
// ===========================================================================

// Symbols one lane stages at most: 8 automaton entries of <= 4 plus the code
// open at bit 64 (an exact-path chunk is capped at the same number), i.e.
// 132 bits; the spill dwords after each staging buffer hold that much past
// a start clamped to the buffer's end.
constexpr int kMaxLaneSyms = 8 * kDfaMaxSyms + 1;
constexpr int kSpillDwords = 8;

// The reference rule (decode.cu:85-112) over one chunk, symbol by symbol,
// from its gap: f(v) for each symbol starting before bit 64; a code-less
// LUT entry ends the chunk.  LUT reads go to global memory (rare path).
template <class F>
__device__ __forceinline__ void exact_walk(const uint3 &d, uint32_t gap,
                                           const uint8_t *__restrict__ luts, int n_luts, F &&f) {
  // a chunk of codes >= 2 bits owns at most 32; the cap bounds what a
  // corrupt table's exact row could make the staging ORs reach
  int left = kMaxLaneSyms;
  // opaque copies: keeps the byte swaps inside the caller's (rare) branch
  // instead of hoisted into the common path
  uint32_t dx = d.x, dy = d.y, dz = d.z;
  asm volatile("" : "+v"(dx), "+v"(dy), "+v"(dz));
  const uint64_t hi = __builtin_bswap64(((uint64_t)dy << 32) | dx);
  const uint32_t la = ((dz & 0xFFu) << 8) | ((dz >> 8) & 0xFFu);
  const uint32_t len_row = (uint32_t)(n_luts - 1) * 256;
  const uint32_t max_row = (uint32_t)(n_luts - 2);
  for (int q = (int)gap; q < kChunkBits;) {
    const uint64_t w = q < 48 ? (hi << q) : (((hi << 32) | ((uint64_t)la << 16)) << (q - 32));
    const uint32_t w16 = (uint32_t)(w >> 48);
    uint32_t v = luts[w16 >> 8];
    if (v >= 240) v = luts[min(256 - v, max_row) * 256 + (w16 & 0xFF)];
    const uint32_t len = luts[len_row + v];
    if (len == 0 || left-- == 0) break;
    f(v & 0xFu);
    q += (int)len;
  }
}


// One compressed block's device buffers.
struct BlockArgs {
  const uint8_t *luts;
  int n_luts;
  const uint8_t *encoded;
  uint32_t n_bytes;
  const uint8_t *packed;
  const uint32_t *op32;  // output_positions as little-endian dword pairs
  const uint8_t *gaps;
  uint8_t *out;
  uint32_t n_elements;
  // scaled bf16 output instead of out (ecf8_decode_bf16)
  uint16_t *out16 = nullptr;
  const ScalePart *parts = nullptr;  // LDS copy of the part table
  int n_parts = 0;
};

// Decode format-blocks fb, fb + fb_step, ... below fb_end (fb < fb_end) of
// one tensor whose table is in s_dfa (loaded before the first barrier here).
// s_edge's slots must be empty on entry; they are empty again on return, and
// every wave has passed a final barrier.
//
// kChecked: tensors too small for the clamped vector loads (fewer than 12
// bitstream bytes or 16 elements) use byte-wise loads throughout.
//
// load_table (optional): a table to load into s_dfa first -- after the
// first block's loads are issued, so the two round trips overlap.
template <int kThreads, bool kChecked, bool kPrio = true, bool kBf16 = false>
__device__ __forceinline__ void dfa_blocks(const BlockArgs &a, uint32_t *s_dfa,
                                           int *s_wave_sum, uint32_t *s_edge, uint32_t *s_dyn,
                                           int stage_cap, int fb, int fb_step, int fb_end,
                                           const uint32_t *load_table = nullptr) {
  constexpr int kWaves = kThreads / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int stage_dw = stage_dwords(stage_cap);
  const int stage_stride = stage_dw + kSpillDwords;
  const uint8_t *const luts = a.luts;
  const int n_luts = a.n_luts;
  const uint8_t *const encoded = a.encoded;
  const uint32_t n_bytes = a.n_bytes;
  const uint8_t *const packed = a.packed;
  const uint32_t *const op32 = a.op32;
  const uint8_t *const gaps = a.gaps;
  uint8_t *const out = a.out;
  const uint32_t n_elements = a.n_elements;

  const uint32_t last12 = kChecked ? 0u : ((n_bytes - 12) & ~7u);
  const uint32_t last8 = kChecked ? 0u : (((n_elements >> 1) - 8) & ~7u);
  const uint32_t last4 = kChecked ? 0u : (((n_elements >> 1) - 4) & ~3u);

  auto fetch = [&](int fb_) {
    const uint32_t g = (uint32_t)fb_ * kThreads + tid;
    RawChunk r;
    if (kChecked) {
      r.v = u32x3_a8{0u, 0u, 0u};
      r.gap_byte = gaps[g >> 1];
    } else {
      r = fetch_chunk(encoded, last12, gaps, g);
    }
    return r;
  };
  uint32_t g_cur = (uint32_t)fb * kThreads + tid;
  const RawChunk raw0 = fetch(fb);
  uint3 cur = chunk_bytes(raw0, encoded, n_bytes, g_cur, !kChecked);
  uint32_t gap = gap_of(raw0.gap_byte, g_cur);
  // This block's output range, wave-uniform.  Positions are below 2^31
  // (checked on the host), so only the low dword of each little-endian u64
  // is loaded: a dead high half would be reused as a temporary and force an
  // early wait on every load in flight.  Positions are always read (readlane
  // waits on the vector load) before the block's stores are issued: the
  // memory counter also counts stores, so a later wait would drain them too.
  uint32_t op_lo, op_hi;
  {
    const uint32_t opv = op32[2 * (fb + (lane & 1))];
    if (load_table) load_dfa_rounds<kThreads, 7>(s_dfa, load_table, tid);
    op_lo = __builtin_amdgcn_readlane(opv, 0);
    op_hi = __builtin_amdgcn_readlane(opv, 1);
  }
  __syncthreads();

  for (int buf_sel = 0;; buf_sel ^= 1) {
    uint32_t *const stage = s_dyn + buf_sel * stage_stride;
    const int fb_next = fb + fb_step;
    // prefetch target: the next block, or this one again after the last (in
    // bounds, discarded) so no load or wait depends on a branch
    const int fb_pf = fb_next < fb_end ? fb_next : fb;

    const BlockRange br = block_range(op_lo, op_hi, n_elements, stage_cap);
    uint2 pre0 = make_uint2(0, 0), pre1 = make_uint2(0, 0);
    uint32_t preh[kHalfPrefetch] = {};
    if constexpr (kBf16) prefetch_nibbles_half(br, packed, last4, tid, kThreads, preh);
    else if (!kChecked) prefetch_nibbles(br, packed, last8, tid, kThreads, pre0, pre1);
    // the next block's chunk and positions (vector loads, so the LDS waits
    // below never wait on them)
    const RawChunk nxt_raw = fetch(fb_pf);
    const uint32_t nopv = op32[2 * (fb_pf + (lane & 1))];

    for (int i = tid; i < ((br.seg_dw + 3) >> 2); i += kThreads)
      reinterpret_cast<uint4 *>(stage)[i] = make_uint4(0, 0, 0, 0);

    // Wave priorities rise with the phase (lookups 0, prefix and staging 1,
    // stores 2): on a CU shared by 4 workgroups, the one furthest along its
    // block issues first, so blocks finish and their stores leave sooner
    // instead of every workgroup's lookups competing on equal terms.
    // Measured on MI355X: 76.4 -> 72.8 us per Qwen3-8B layer.
    if (kPrio) __builtin_amdgcn_s_setprio(0);
    // ---- 1. the byte automaton over this lane's chunk.  The first code
    // starts at bit `gap`: inside byte 0 (start from the skip-`gap` row) or
    // inside byte 1 (byte 0 is skipped whole, then `gap - 8` bits).
    const uint32_t a0 = gap < 8 ? ((gap << 10) | ((cur.x << 2) & 0x3FCu))
                                : (uint32_t)(kDfaSkipByte * 4) + ((gap - 8) << 2);
    const uint32_t e0 = dfa_at(s_dfa, a0);
    const uint32_t e1 = dfa_at(s_dfa, (e0 & kDfaRowMask) | ((cur.x >> 6) & 0x3FCu));
    const uint32_t e2 = dfa_at(s_dfa, (e1 & kDfaRowMask) | ((cur.x >> 14) & 0x3FCu));
    const uint32_t e3 = dfa_at(s_dfa, (e2 & kDfaRowMask) | ((cur.x >> 22) & 0x3FCu));
    const uint32_t e4 = dfa_at(s_dfa, (e3 & kDfaRowMask) | ((cur.y << 2) & 0x3FCu));
    const uint32_t e5 = dfa_at(s_dfa, (e4 & kDfaRowMask) | ((cur.y >> 6) & 0x3FCu));
    const uint32_t e6 = dfa_at(s_dfa, (e5 & kDfaRowMask) | ((cur.y >> 14) & 0x3FCu));
    const uint32_t e7 = dfa_at(s_dfa, (e6 & kDfaRowMask) | ((cur.y >> 22) & 0x3FCu));
    // A code still open at bit 64 started in this chunk, so it is owned
    // here: its symbol is the first one completed in the look-ahead bytes
    // (codes are at most 16 bits, so it ends in byte 8 or 9).
    const uint32_t row7 = e7 & kDfaRowMask;
    const bool open = row7 >= ((uint32_t)kDfaFirstPendingRow << 10);
    uint32_t e8 = dfa_at(s_dfa, row7 | ((cur.z << 2) & 0x3FCu));
    if (__builtin_amdgcn_ballot_w64(open && (e8 & 0xFFu) == 0)) {
      const uint32_t e9 = dfa_at(s_dfa, (e8 & kDfaRowMask) | ((cur.z >> 6) & 0x3FCu));
      if ((e8 & 0xFFu) == 0) e8 = e9;
    }
    const uint32_t et = open ? ((e8 & 0xF0000u) | 4u) : 0u;
    // symbol counts are kept x4: the width of the chunk's nibbles in bits
    int cnt4 = (int)((e0 & 0xFFu) + (e1 & 0xFFu) + (e2 & 0xFFu) + (e3 & 0xFFu) + (e4 & 0xFFu) +
                     (e5 & 0xFFu) + (e6 & 0xFFu) + (e7 & 0xFFu) + (et & 0xFFu));
    // lanes in the exact row (the stream's final padding) count their chunk
    // with the reference rule instead
    const bool exact = row7 == ((uint32_t)kDfaExactRow << 10);
    const bool any_exact = __builtin_amdgcn_ballot_w64(exact) != 0;
    if (any_exact && exact) {
      int n = 0;
      exact_walk(cur, gap, luts, n_luts, [&](uint32_t) { ++n; });
      cnt4 = 4 * n;
    }

    if (kPrio) __builtin_amdgcn_s_setprio(1);
    // ---- 2. block-wide exclusive prefix of the per-chunk symbol counts
    const int incl = wave_inclusive_scan(cnt4);
    if (lane == 63) s_wave_sum[wave] = incl;
    __syncthreads();
    const int excl4 = incl - cnt4 + waves_before<kWaves>(s_wave_sum, lane, wave);
    // the previous block's edge segments (parked before the barrier above)
    if constexpr (kBf16) flush_edges_bf16(s_edge, a.out16, tid, kThreads - 64);
    else flush_edges(s_edge, out, tid, kThreads - 64);
    // bf16 output: the scales of this lane's first two segments, loaded
    // while the staging ORs run (positions clamped into the tensor, so every
    // lookup is in bounds; lanes past the block's segments discard theirs)
    float sc[kScalePrefetch] = {};
    int k0 = 0;
    if constexpr (kBf16) {
      const uint32_t last_half = n_elements - 8u;
      // the block's first part; lanes past the block's outputs look up a
      // scale at a clamped position and discard it
      k0 = __builtin_amdgcn_readfirstlane(part_of(a.parts, a.n_parts, min(br.base, last_half)));
#pragma unroll
      for (int k = 0; k < kScalePrefetch; ++k)
        sc[k] = segment_scale(a.parts, a.n_parts, k0,
                              min(br.base + 8u * (uint32_t)(tid + k * kThreads), last_half));
    }

    // ---- 3. OR the exponents into the staging buffer at their positions,
    // two automaton entries (at most 8 symbols, 32 bits) per 64-bit OR.
    // Symbols past the block's count (only the stream's last chunk decodes
    // any: padding) land past the block's outputs and are never stored;
    // positions past the buffer go to its spill dwords.
    // A lane's ORs reach at most 33 symbols (132 bits) past its start, so a
    // start clamped to the buffer's end keeps every OR inside the buffer's
    // 8 spill dwords (reached only by positions past the block's count).
    uint32_t pos4 = min(((uint32_t)br.lead << 2) + (uint32_t)excl4, (uint32_t)stage_dw << 5);
    auto put = [&](uint32_t syms, uint32_t n4) {
      const uint64_t v = (uint64_t)syms << (pos4 & 31u);
      uint32_t *const q = stage + __builtin_amdgcn_ubfe(pos4, 5, 27);
      atomicOr(q, (uint32_t)v);
      atomicOr(q + 1, (uint32_t)(v >> 32));
      pos4 += n4;
    };
    auto put2 = [&](uint32_t ea, uint32_t eb) {
      // (eb.hi16 << count4(ea)) | ea.hi16 in two SDWA ops (count4 <= 16, so
      // the whole dword is a valid shift amount)
      uint32_t t, syms;
      asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
          "src1_sel:WORD_1"
          : "=v"(t) : "v"(ea), "v"(eb));
      asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
          "src1_sel:WORD_1"
          : "=v"(syms) : "v"(t), "v"(ea));
      put(syms, (ea & 0xFFu) + (eb & 0xFFu));
    };
    if (!any_exact || !exact) {
      put2(e0, e1);
      put2(e2, e3);
      put2(e4, e5);
      put2(e6, e7);
      put(et >> 16, 0u);
    } else {  // at most 32 codes of >= 2 bits start in the chunk
      exact_walk(cur, gap, luts, n_luts, [&](uint32_t v) { put(v, 4u); });
    }
    __syncthreads();

    // ---- 4. merge with the sign/mantissa nibbles and store FP8 bytes
    if (kPrio) __builtin_amdgcn_s_setprio(2);
    if constexpr (kBf16)
      write_block_bf16<kThreads>(stage, br, preh, sc, packed, n_elements, a.out16, s_edge, tid,
                                 a.parts, a.n_parts, k0);
    else
      write_block<kThreads, kChecked>(stage, br, pre0, pre1, packed, n_elements, out, s_edge,
                                      tid);
    if (kPrio) __builtin_amdgcn_s_setprio(0);
    // the next iteration writes the other staging buffer; its barrier after
    // the scan orders this sweep before any reuse of this one
    if (fb_next >= fb_end) break;
    // The next block's chunk and positions, fetched a whole decode phase
    // ago, are read only now, after this block's stores were issued: the
    // memory counter also counts stores, and waiting for a load waits for
    // every older store too.  Here the only older stores are the previous
    // block's, issued an iteration ago; read before the stores above, the
    // wait would have drained them mid-iteration.
    g_cur = (uint32_t)fb_pf * kThreads + tid;
    cur = chunk_bytes(nxt_raw, encoded, n_bytes, g_cur, !kChecked);
    gap = gap_of(nxt_raw.gap_byte, g_cur);
    op_lo = __builtin_amdgcn_readlane(nopv, 0);
    op_hi = __builtin_amdgcn_readlane(nopv, 1);
    fb = fb_next;
  }
  __syncthreads();
  if constexpr (kBf16) flush_edges_bf16(s_edge, a.out16, tid, kThreads - 64);
  else flush_edges(s_edge, out, tid, kThreads - 64);
}

// One tensor: the persistent grid strides over its format-blocks.
//
// SGPRs are capped at 80: measured on MI355X, above that fewer than 8 waves
// per SIMD fit (3 workgroups of 512 per CU instead of 4); the few spills
// the cap causes go to VGPR lanes.
// kKindCheck: the table's kind is only known on the device (built there by
// ecf8_build_table); the grid exits unless the table is an automaton.
template <int kThreads, bool kChecked, bool kKindCheck>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_num_sgpr(80), amdgpu_waves_per_eu(8))) void decode_dfa_kernel(
    const uint8_t *__restrict__ luts, int n_luts, const uint32_t *__restrict__ table,
    const uint8_t *__restrict__ encoded, uint32_t n_bytes,
    const uint8_t *__restrict__ packed, const uint64_t *__restrict__ op,
    const uint8_t *__restrict__ gaps, uint8_t *__restrict__ out, uint32_t n_elements, int n_fb,
    int stage_cap) {
  constexpr int kWaves = kThreads / 64;
  __shared__ uint32_t s_dfa[kDfaEntries];
  __shared__ int s_wave_sum[kWaves];
  __shared__ __attribute__((aligned(16))) uint32_t s_edge[kEdgeDwords];
  // dynamic LDS: 2 staging buffers, each followed by kSpillDwords spill
  // dwords that take the ORs of positions past the buffer
  extern __shared__ __attribute__((aligned(16))) uint32_t s_dyn[];

  if (kKindCheck && table[kDfaEntries] != (uint32_t)ECF8_TABLE_DFA) return;  // uniform
  const int tid = threadIdx.x;
  load_dfa_batched<kThreads>(s_dfa, table, tid);
  if (tid < kEdgeDwords) s_edge[tid] = 0u;
  if ((int)blockIdx.x >= n_fb) return;  // uniform per workgroup, before any barrier
  const BlockArgs a{luts, n_luts, encoded, n_bytes, packed,
                    reinterpret_cast<const uint32_t *>(op), gaps, out, n_elements};
  dfa_blocks<kThreads, kChecked>(a, s_dfa, s_wave_sum, s_edge, s_dyn, stage_cap,
                                 (int)blockIdx.x, (int)gridDim.x, n_fb);
}

// One tensor decoded into scaled bf16 (ecf8_decode_bf16): the DFA kernel's
// grid and phases, with each 16-element segment converted by its part's
// block scale before the store.  The part table is copied into LDS (parts.n
// <= ECF8_MAX_SCALED_PARTS entries, checked on the host).
template <int kThreads>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_num_sgpr(80), amdgpu_waves_per_eu(8))) void decode_dfa_bf16_kernel(
    const uint8_t *__restrict__ luts, int n_luts, const uint32_t *__restrict__ table,
    const uint8_t *__restrict__ encoded, uint32_t n_bytes,
    const uint8_t *__restrict__ packed, const uint64_t *__restrict__ op,
    const uint8_t *__restrict__ gaps, uint16_t *__restrict__ out16, uint32_t n_elements,
    int n_fb, int stage_cap, const ScaleParts parts) {
  constexpr int kWaves = kThreads / 64;
  __shared__ uint32_t s_dfa[kDfaEntries];
  __shared__ int s_wave_sum[kWaves];
  __shared__ __attribute__((aligned(16))) uint32_t s_edge[kEdgeDwords];
  __shared__ ScalePart s_parts[ECF8_MAX_SCALED_PARTS];
  extern __shared__ __attribute__((aligned(16))) uint32_t s_dyn[];

  const int tid = threadIdx.x;
  load_dfa_batched<kThreads>(s_dfa, table, tid);
  if (tid < kEdgeDwords) s_edge[tid] = 0u;
  if (tid < parts.n) s_parts[tid] = parts.p[tid];
  if ((int)blockIdx.x >= n_fb) return;  // uniform per workgroup, before any barrier
  BlockArgs a{luts, n_luts, encoded, n_bytes, packed,
              reinterpret_cast<const uint32_t *>(op), gaps, nullptr, n_elements};
  a.out16 = out16;
  a.parts = s_parts;
  a.n_parts = parts.n;
  dfa_blocks<kThreads, false, true, true>(a, s_dfa, s_wave_sum, s_edge, s_dyn, stage_cap,
                                          (int)blockIdx.x, (int)gridDim.x, n_fb);
}

// Routed launches over at most this many tensors (e.g. an MoE layer's
// attention block and 128 experts) select on the device in the batched
// kernel itself (kSelect): each workgroup scans the selected tensors' task
// counts into an LDS task table and finds a task's tensor there, so no
// compaction kernel runs first.  Whole launches keep the binary search over
// the descriptors' task_begin, in their own instance: compiled into one
// kernel, the table's code raised its register spills, and on MI355X a
// whole Qwen3-30B-A3B layer then fetched ~17 MB more per launch beyond L2
// and ran 0.3 % slower.
constexpr int kLdsBlocks = 256;

// Many tensors in one launch (e.g. the routed experts of an MoE layer): the
// work is split into tasks of up to `blocks_per_task` format-blocks of one
// tensor; desc[d].task_begin is the first task of tensor d.  Each workgroup
// takes tasks blockIdx.x, + gridDim.x, ..., loading the task's table before
// decoding it.
//
// kSelect (count <= kLdsBlocks): select holds one flag per descriptor; only
// the tensors whose flag is nonzero are decoded, their tasks numbered in
// descriptor order (task_begin is then ignored), and workgroup 0 writes
// {selected tensors, their tasks} to sel_counts (optional).
// dev_counts (optional, with descriptors compacted by select_blocks_kernel):
// {count, n_tasks} read from device memory instead of the arguments.
template <int kThreads, bool kSelect>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_num_sgpr(80), amdgpu_waves_per_eu(8))) void decode_dfa_batched_kernel(
    const ecf8_block_desc *__restrict__ descs, int count, int n_tasks, int blocks_per_task,
    int stage_cap, const int *__restrict__ dev_counts, const int32_t *__restrict__ select,
    int32_t *__restrict__ sel_counts) {
  constexpr int kWaves = kThreads / 64;
  static_assert(kLdsBlocks == 4 * 64, "one 16-byte read of the task table per lane");
  constexpr int kTable = kSelect ? kLdsBlocks : 4;  // the whole-launch instance keeps none
  __shared__ uint32_t s_dfa[kDfaEntries];
  __shared__ int s_wave_sum[kWaves];
  __shared__ __attribute__((aligned(16))) uint32_t s_edge[kEdgeDwords];
  __shared__ __attribute__((aligned(16))) int s_begin[kTable];
  __shared__ int s_wave_sel[kSelect ? kWaves : 1];
  extern __shared__ __attribute__((aligned(16))) uint32_t s_dyn[];

  if (dev_counts) {  // never above the launch's bounds
    count = min(count, __builtin_amdgcn_readfirstlane(dev_counts[0]));
    n_tasks = min(n_tasks, __builtin_amdgcn_readfirstlane(dev_counts[1]));
  }
  const int tid = threadIdx.x;
  if (tid < kEdgeDwords) s_edge[tid] = 0u;
  constexpr uint32_t kBlockBytes = (uint32_t)kThreads * kChunkBytes;
  if constexpr (kSelect) {
    const int lane = tid & 63, wave = tid >> 6;
    // s_begin[b]: tensor b's first task (an exclusive prefix of the
    // selected tensors' task counts, computed as the descriptors' task_begin
    // is); past the last tensor INT32_MAX, so that the search below never
    // picks those entries.  Both loads of a tensor are issued together.
    int base = 0, n_sel = 0;
    for (int c0 = 0; c0 < kLdsBlocks; c0 += kThreads) {  // one pass for >= 256 threads
      const int b = c0 + tid;
      int tasks = 0, flag = 0;
      if (b < count) {
        flag = select[b];
        const int64_t nb = min(max(descs[b].n_bytes, (int64_t)0), (int64_t)INT32_MAX);
        const int fbs = (int)((nb + kBlockBytes - 1) / kBlockBytes);
        tasks = flag != 0 ? (fbs + blocks_per_task - 1) / blocks_per_task : 0;
      }
      const int incl = wave_inclusive_scan(tasks);
      const int wave_sel = __builtin_popcountll(__builtin_amdgcn_ballot_w64(flag != 0));
      if (lane == 63) {
        s_wave_sum[wave] = incl;
        s_wave_sel[wave] = wave_sel;
      }
      __syncthreads();
      int total = 0;
      const int before = waves_before<kWaves>(s_wave_sum, lane, wave, &total);
      if (b < kLdsBlocks) s_begin[b] = b < count ? base + before + incl - tasks : INT32_MAX;
      if (sel_counts && tid == 0)
        for (int w = 0; w < kWaves; ++w) n_sel += s_wave_sel[w];
      base += total;
      __syncthreads();  // s_wave_sum is written again by the next pass and the decode
    }
    n_tasks = min(n_tasks, base);
    if (sel_counts && blockIdx.x == 0 && tid == 0) {
      sel_counts[0] = n_sel;
      sel_counts[1] = base;
    }
  } else {
    (void)select;
    (void)sel_counts;
  }
  // Task order.  Several tensors: the workgroups of XCD x (workgroups are
  // dealt to the 8 XCDs round robin) take the x-th eighth of the task list,
  // strided over them, so a tensor's tasks share one XCD's L2 and its table
  // is fetched from HBM about once instead of once per XCD.  One tensor, or
  // a grid that is not a multiple of 8: tasks strided over the whole grid.
  constexpr int kXcds = 8;
  int task = blockIdx.x, task_end = n_tasks, task_step = gridDim.x;
  if (count > 1 && gridDim.x % kXcds == 0) {
    const int x = blockIdx.x % kXcds, per = gridDim.x / kXcds;
    task = (int)(((int64_t)x * n_tasks) / kXcds) + (int)(blockIdx.x / kXcds);
    task_end = (int)(((int64_t)(x + 1) * n_tasks) / kXcds);
    task_step = per;
  }
  for (; task < task_end; task += task_step) {
    // the tensor of this task: the last descriptor whose first task is <= it
    int lo = 0, first = 0;
    if constexpr (kSelect) {
      // first tasks ascend: those <= task are a prefix of the table, counted
      // with one ballot per entry of each lane's four
      const int4 v = reinterpret_cast<const int4 *>(s_begin)[threadIdx.x & 63];
      const int n = __builtin_popcountll(__builtin_amdgcn_ballot_w64(v.x <= task)) +
                    __builtin_popcountll(__builtin_amdgcn_ballot_w64(v.y <= task)) +
                    __builtin_popcountll(__builtin_amdgcn_ballot_w64(v.z <= task)) +
                    __builtin_popcountll(__builtin_amdgcn_ballot_w64(v.w <= task));
      if (n == 0) continue;  // uniform; never for a task below n_tasks
      lo = n - 1;
      first = __builtin_amdgcn_readfirstlane(s_begin[lo]);
    } else {
      int hi = count - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (descs[mid].task_begin <= task) lo = mid;
        else hi = mid - 1;
      }
      first = descs[lo].task_begin;
    }
    const ecf8_block_desc &d = descs[lo];
    // uniform; blocks too small for the clamped vector loads (fewer than 12
    // bitstream bytes or 16 elements) or too large for 32-bit positions are
    // not batched, nor is a task outside its block (malformed task_begin)
    if (d.n_bytes < 12 || d.n_elements < 16 || d.n_bytes > INT32_MAX - 64 ||
        d.n_elements > INT32_MAX - 64 || task < first)
      continue;
    const uint32_t n_bytes = (uint32_t)d.n_bytes;
    const int n_fb = (int)((n_bytes + kBlockBytes - 1) / kBlockBytes);
    // A tensor's tasks interleave its format-blocks (task r takes r,
    // r + tasks, ...): its tasks run at the same time on one XCD (the order
    // above), so together they sweep the tensor's bytes in order, as the
    // one-tensor kernel's grid does.  Measured on MI355X, a whole
    // Qwen3-30B-A3B layer (two rotated sets): 245.5 us with contiguous runs
    // of blocks per task, 238.6 us interleaved.
    const int tasks = (n_fb + blocks_per_task - 1) / blocks_per_task;
    const int r = task - first;
    if (r >= tasks) continue;
    // the previous task ended with a barrier: no wave still reads s_dfa.
    // The table loads in dfa_blocks, seven per lane in flight (two round
    // trips instead of thirteen), overlapped with the first block's.
    const BlockArgs a{as_global(d.luts), d.n_luts, as_global(d.encoded), n_bytes,
                      as_global(d.packed_other_4bits),
                      as_global(reinterpret_cast<const uint32_t *>(d.output_positions)),
                      as_global(d.gaps), as_global(d.outputs), (uint32_t)d.n_elements};
    dfa_blocks<kThreads, false>(a, s_dfa, s_wave_sum, s_edge, s_dyn, stage_cap, r, tasks, n_fb,
                                as_global(d.table));
  }
}

// Compact the descriptors whose select flag is nonzero (e.g. the attention
// block and the experts the router picked this step) into `out`, in order,
// with task_begin recomputed for the compacted list, and write {count,
// n_tasks} to `counts` for decode_dfa_batched_kernel.  One workgroup of
// 1024 threads walks the descriptors in chunks of 1024.
__global__ __launch_bounds__(1024) void select_blocks_kernel(
    const ecf8_block_desc *__restrict__ in, int count, const int32_t *__restrict__ select,
    int blocks_per_task, int64_t block_bytes, ecf8_block_desc *__restrict__ out,
    int *__restrict__ counts) {
  constexpr int kWaves = 16;
  __shared__ int s_sel[kWaves], s_task[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int base_sel = 0, base_task = 0;
  for (int c0 = 0; c0 < count; c0 += 1024) {
    const int d = c0 + tid;
    int sel = 0, tasks = 0;
    if (d < count && select[d] != 0) {
      const int64_t nb = in[d].n_bytes > 0 ? in[d].n_bytes : 0;
      const int64_t n_fb = (nb + block_bytes - 1) / block_bytes;
      sel = 1;
      tasks = (int)((n_fb + blocks_per_task - 1) / blocks_per_task);
    }
    const int isel = wave_inclusive_scan(sel), itask = wave_inclusive_scan(tasks);
    if (lane == 63) {
      s_sel[wave] = isel;
      s_task[wave] = itask;
    }
    __syncthreads();
    int total_sel = 0, total_task = 0;
    const int before_sel = waves_before<kWaves>(s_sel, lane, wave, &total_sel);
    const int before_task = waves_before<kWaves>(s_task, lane, wave, &total_task);
    if (sel) {
      ecf8_block_desc e = in[d];
      e.task_begin = base_task + before_task + itask - tasks;
      out[base_sel + before_sel + isel - 1] = e;
    }
    base_sel += total_sel;
    base_task += total_task;
    __syncthreads();  // the totals are rewritten by the next chunk
  }
  if (tid == 0) {
    counts[0] = base_sel;
    counts[1] = base_task;
  }
}

// ===========================================================================
// MULTI kernel (tables of kind ECF8_TABLE_MULTI)
// ===========================================================================

// The chunk as a big-endian bit string (hi), its two look-ahead bytes (la)
// and its gap.
struct Chunk {
  uint64_t hi;
  uint32_t la;
  uint32_t gap;
};

__device__ __forceinline__ Chunk finish_chunk(const RawChunk &r, const uint8_t *__restrict__ encoded,
                                              uint32_t n_bytes, uint32_t g, bool vector_ok) {
  const uint3 d = chunk_bytes(r, encoded, n_bytes, g, vector_ok);
  Chunk c;
  c.hi = __builtin_bswap64(((uint64_t)d.y << 32) | d.x);
  c.la = ((d.z & 0xFFu) << 8) | ((d.z >> 8) & 0xFFu);
  c.gap = gap_of(r.gap_byte, g);
  return c;
}

// Bits [p, p+16) of the 80-bit string hi:la (chunk + look-ahead), p < 64.
__device__ __forceinline__ uint32_t window16(uint64_t hi, uint32_t la, int p) {
  const uint64_t w = p < 48 ? (hi << p) : (((hi << 32) | ((uint64_t)la << 16)) << (p - 32));
  return (uint32_t)(w >> 48);
}

// Dwords of a lane's nibble run: room for every symbol a chunk can own when
// no code is shorter than min_bits, plus the spill dword of the last 64-bit OR.
__host__ __device__ constexpr int run_slots_for(int min_bits) {
  return ((kChunkBits + min_bits - 1) / min_bits + 7) / 8 + 1;
}
constexpr int kZeroEntry = kMultiEntries;  // all-zero table entry: a lookup that does nothing

// kKindCheck: as for decode_dfa_kernel, the grid exits unless the table is
// a multi-symbol table.
template <int kThreads, bool kChecked, bool kKindCheck>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_num_sgpr(80))) void decode_multi_kernel(
    const uint8_t *__restrict__ luts, int n_luts, const uint32_t *__restrict__ table,
    const uint8_t *__restrict__ encoded, uint32_t n_bytes, const uint8_t *__restrict__ packed,
    const uint64_t *__restrict__ op, const uint8_t *__restrict__ gaps,
    uint8_t *__restrict__ out, uint32_t n_elements, int n_fb, int stage_cap, int run_slots) {
  constexpr int kWaves = kThreads / 64;
  // dynamic LDS: [run_slots][kThreads] nibble runs, then 2 staging buffers
  extern __shared__ __attribute__((aligned(16))) uint32_t s_dyn[];
  __shared__ uint32_t s_table[kMultiEntries + 1];
  __shared__ int s_wave_sum[kWaves];
  __shared__ __attribute__((aligned(16))) uint32_t s_edge[kEdgeDwords];

  if (kKindCheck && table[kDfaEntries] != (uint32_t)ECF8_TABLE_MULTI) return;  // uniform
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int stage_dw = stage_dwords(stage_cap);
  uint32_t *const s_stage = s_dyn + run_slots * kThreads;
  uint32_t *const run = s_dyn + tid;  // slot k at run[k * kThreads]
  const int max_slot = run_slots - 2;  // last slot a 64-bit OR may start in

  {  // all of a lane's table loads in flight before the first wait
    constexpr int kIters = (kMultiEntries + 1 + kThreads - 1) / kThreads;
    constexpr int kBatch = kIters < 13 ? kIters : 13;
#pragma unroll
    for (int j0 = 0; j0 < kIters; j0 += kBatch) {
      uint32_t v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = tid + (j0 + j) * kThreads;
        v[j] = i < kMultiEntries ? table[i] : 0u;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = tid + (j0 + j) * kThreads;
        if (i <= kMultiEntries) s_table[i] = v[j];
      }
    }
  }
  if (tid < kEdgeDwords) s_edge[tid] = 0u;
  const int len_row = (n_luts - 1) * 256;
  const uint32_t max_row = (uint32_t)(n_luts - 2);

  int fb = blockIdx.x;
  if (fb >= n_fb) return;  // uniform per workgroup, before any barrier
  const uint32_t last12 = kChecked ? 0u : ((n_bytes - 12) & ~7u);
  const uint32_t last8 = kChecked ? 0u : (((n_elements >> 1) - 8) & ~7u);

  auto fetch = [&](int fb_) {
    const uint32_t g = (uint32_t)fb_ * kThreads + tid;
    RawChunk r;
    if (kChecked) {
      r.v = u32x3_a8{0u, 0u, 0u};
      r.gap_byte = gaps[g >> 1];
    } else {
      r = fetch_chunk(encoded, last12, gaps, g);
    }
    return r;
  };
  Chunk cur = finish_chunk(fetch(fb), encoded, n_bytes, (uint32_t)fb * kThreads + tid, !kChecked);
  const uint32_t *const op32 = reinterpret_cast<const uint32_t *>(op);
  uint32_t op_lo, op_hi;
  {
    const uint32_t opv = op32[2 * (fb + (lane & 1))];
    op_lo = __builtin_amdgcn_readlane(opv, 0);
    op_hi = __builtin_amdgcn_readlane(opv, 1);
  }
  __syncthreads();

  for (int buf_sel = 0;; buf_sel ^= 1) {
    uint32_t *const stage = s_stage + buf_sel * stage_dw;
    const int fb_next = fb + (int)gridDim.x;
    const int fb_pf = fb_next < n_fb ? fb_next : fb;

    const BlockRange br = block_range(op_lo, op_hi, n_elements, stage_cap);
    const int total = (int)(br.end - br.start);
    uint2 pre0 = make_uint2(0, 0), pre1 = make_uint2(0, 0);
    if (!kChecked) prefetch_nibbles(br, packed, last8, tid, kThreads, pre0, pre1);
    const RawChunk nxt_raw = fetch(fb_pf);
    const uint32_t nopv = op32[2 * (fb_pf + (lane & 1))];

    // ---- 1. decode the codes this lane's chunk owns into its nibble run
    for (int k = 0; k < run_slots; ++k) run[k * kThreads] = 0u;
    for (int i = tid; i < ((br.seg_dw + 3) >> 2); i += kThreads)
      reinterpret_cast<uint4 *>(stage)[i] = make_uint4(0, 0, 0, 0);

    int p = (int)cur.gap;              // bit offset of the next code in the chunk
    uint64_t buf = cur.hi << cur.gap;  // the bits from p on, left-aligned
    int cnt = 0;                       // exponents in the run
    // OR an entry's exponents (its unused nibbles are zero) at nibble cnt of
    // the run; nibbles past the counted ones are masked off by the copy
    auto emit = [&](uint32_t e, uint32_t n) {
      const uint64_t v = (uint64_t)(e & 0xFFFFu) << ((cnt & 7) * 4);
      // runs are sized for the block's shortest code; the clamp only keeps
      // LDS accesses in bounds for inputs that break that bound
      uint32_t *q = run + min(cnt >> 3, max_slot) * kThreads;
      atomicOr(q, (uint32_t)v);
      atomicOr(q + kThreads, (uint32_t)(v >> 32));
      cnt += (int)n;
    };
    // A lookup at a code longer than the 12-bit window reads an all-zero
    // entry: the lane emits nothing and stays in place ("parked") until the
    // exact path below.  Codes starting before bit 53 have 12 valid window
    // bits and all their entry's symbols end inside the chunk.  Every lane
    // starts below bit 16 and a lookup spans at most 12 bits, so the first
    // four lookups need no predicate.
    uint32_t e = 1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      e = s_table[(uint32_t)(buf >> 52)];
      const uint32_t len = entry_len(e);
      emit(e, __builtin_popcount(entry_mask(e)));
      p += (int)len;
      buf <<= len;
    }
    // then while any lane of the wave is active; inactive lanes read the
    // zero entry, which changes nothing.  A lane stops at an entry of length
    // 0 whatever its other bits (a corrupt table cannot stall the loop).
    bool act = entry_len(e) != 0 && p < 53;
    while (__builtin_amdgcn_ballot_w64(act)) {
      e = s_table[act ? (uint32_t)(buf >> 52) : (uint32_t)kZeroEntry];
      const uint32_t len = entry_len(e);
      emit(e, __builtin_popcount(entry_mask(e)));
      p += (int)len;
      buf <<= len;
      act = act && len != 0 && p < 53;
    }
    // codes starting in [53, 64) (lanes that did not park): window rebuilt
    // from chunk bits 32..79; entry symbols starting at or after bit 64
    // belong to the next chunk
    act = p >= 53 && p < kChunkBits;
    if (__builtin_amdgcn_ballot_w64(act)) {
      buf = ((cur.hi << 32) | ((uint64_t)cur.la << 16)) << ((p - 32) & 63);
      while (__builtin_amdgcn_ballot_w64(act)) {
        e = s_table[act ? (uint32_t)(buf >> 52) : (uint32_t)kZeroEntry];
        uint32_t len = entry_len(e);
        const uint32_t rem = (uint32_t)(kChunkBits - p) & 31u;  // 1..11 when active
        const uint32_t mask = entry_mask(e);
        const uint32_t kept = mask & ((1u << rem) - 1);
        emit(e, __builtin_popcount(kept));
        len = kept != mask ? rem : len;  // the lane ends at bit 64
        p += (int)len;
        buf <<= (len & 63);
        act = act && len != 0 && p < kChunkBits;
      }
    }
    // parked lanes (a code longer than 12 bits, rare): the exact rule,
    // through the table where it decides and the two-level LUT where not
    if (__builtin_amdgcn_ballot_w64(p < kChunkBits)) {
      if (p < kChunkBits) {
        int q = p;
        while (q < kChunkBits) {
          const uint32_t w16 = window16(cur.hi, cur.la, q);
          uint32_t f = s_table[w16 >> 4];
          uint32_t len = entry_len(f), mask = entry_mask(f);
          if (len == 0) {
            uint32_t v = luts[w16 >> 8];
            if (v >= 240) {
              const uint32_t row = min(256 - v, max_row);
              v = luts[row * 256 + (w16 & 0xFF)];
            }
            len = luts[len_row + v];
            if (len == 0) break;  // code-less entry: only the EOF pad bits reach it
            f = v & 0xF;
            mask = 1;
          }
          const int rem = kChunkBits - q;
          if (rem < kWinBits) {
            const uint32_t kept = mask & ((1u << rem) - 1);
            if (kept != mask) {
              mask = kept;
              len = rem;
            }
          }
          emit(f, __builtin_popcount(mask));
          q += (int)len;
        }
      }
    }

    // ---- 2. block-wide exclusive prefix of the per-chunk symbol counts
    const int incl = wave_inclusive_scan(cnt);
    if (lane == 63) s_wave_sum[wave] = incl;
    __syncthreads();
    const int excl = incl - cnt + waves_before<kWaves>(s_wave_sum, lane, wave);
    flush_edges(s_edge, out, tid, kThreads - 64);

    // ---- 3. OR this lane's nibble run into the staging buffer
    int c = cnt;
    if (excl + c > total) c = total - excl;
    if (c > 0) {
      const int nib0 = br.lead + excl;
      const uint32_t sh = (uint32_t)(nib0 & 7) * 4;
      uint32_t *const dst = stage + (nib0 >> 3);
      const int ndw = min((c + 7) >> 3, run_slots - 1);
      const uint32_t last_mask = (c & 7) ? (1u << (4 * (c & 7))) - 1 : 0xFFFFFFFFu;
      uint32_t carry = 0;
      for (int k = 0; k < ndw; ++k) {
        uint32_t v = run[k * kThreads];
        v &= k == ndw - 1 ? last_mask : 0xFFFFFFFFu;
        const uint64_t w = (uint64_t)v << sh;
        atomicOr(dst + k, (uint32_t)w | carry);
        carry = (uint32_t)(w >> 32);
      }
      if (carry) atomicOr(dst + ndw, carry);
    }
    __syncthreads();

    const Chunk nxt = finish_chunk(nxt_raw, encoded, n_bytes, (uint32_t)fb_pf * kThreads + tid,
                                   !kChecked);
    const uint32_t nop_lo = __builtin_amdgcn_readlane(nopv, 0);
    const uint32_t nop_hi = __builtin_amdgcn_readlane(nopv, 1);

    // ---- 4. merge with the sign/mantissa nibbles and store FP8 bytes
    write_block<kThreads, kChecked>(stage, br, pre0, pre1, packed, n_elements, out, s_edge, tid);
    if (fb_next >= n_fb) break;
    fb = fb_next;
    cur = nxt;
    op_lo = nop_lo;
    op_hi = nop_hi;
  }
  __syncthreads();
  flush_edges(s_edge, out, tid, kThreads - 64);
}

// ===========================================================================
// Launchers
// ===========================================================================

// Per device: CU count, and per kernel variant the occupancy at the last
// dynamic LDS size it was launched with.
// {DFA, MULTI} x 4 block sizes x {unchecked, checked} (slots 0-15), batched
// DFA x 4 (16-19), the device-kind variants of DFA and MULTI (20-35), the
// scaled-bf16 DFA kernel (36), then batched DFA selecting in the kernel x 4
// (37-40)
constexpr int kVariants = 41;
struct LaunchCache {
  int device = -1;
  int cus = 0;
  size_t occ_dyn[kVariants] = {};
  int occ[kVariants] = {};
  bool attr_set[kVariants] = {};
};
constexpr int kMaxDevices = 64;
LaunchCache g_cache[kMaxDevices];

// Grid size for `kernel` (persistent: resident workgroups per CU x CUs).
int persistent_grid(const void *kernel, int threads, size_t dyn, size_t max_dyn, int slot,
                    int64_t n_fb, int *grid) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return ECF8_ERR_HIP;
  LaunchCache &c = g_cache[dev];
  if (c.device != dev || c.cus == 0) {
    if (hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return ECF8_ERR_HIP;
    c.device = dev;
  }
  if (!c.attr_set[slot]) {
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_dyn) !=
        hipSuccess)
      return ECF8_ERR_HIP;
    c.attr_set[slot] = true;
  }
  if (c.occ_dyn[slot] != dyn || c.occ[slot] == 0) {
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, dyn) != hipSuccess)
      return ECF8_ERR_HIP;
    c.occ[slot] = occ > 0 ? occ : 1;
    c.occ_dyn[slot] = dyn;
  }
  const int64_t g = (int64_t)c.cus * c.occ[slot];
  *grid = (int)(g < n_fb ? g : n_fb);
  return ECF8_OK;
}

struct DecodeArgs {
  const uint8_t *luts;
  int n_luts;
  const uint32_t *table;
  const uint8_t *encoded;
  int64_t n_bytes;
  const uint8_t *packed;
  const uint64_t *op;
  const uint8_t *gaps;
  uint8_t *out;
  int64_t n_elements;
  int64_t n_fb;
  int cap;
  int min_code_bits;
  hipStream_t stream;
};

template <int kThreads, bool kChecked, bool kKindCheck>
int launch_dfa(const DecodeArgs &a, int slot) {
  constexpr int kMaxSyms = kThreads * kChunkBits;
  const size_t dyn = sizeof(uint32_t) * 2 * ((size_t)stage_dwords(a.cap) + kSpillDwords);
  const size_t max_dyn = sizeof(uint32_t) * 2 * ((size_t)stage_dwords(kMaxSyms) + kSpillDwords);
  auto kernel = decode_dfa_kernel<kThreads, kChecked, kKindCheck>;
  int grid = 0;
  const int rc = persistent_grid(reinterpret_cast<const void *>(kernel), kThreads, dyn, max_dyn,
                                 slot, a.n_fb, &grid);
  if (rc != ECF8_OK) return rc;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), dyn, a.stream, a.luts,
                     a.n_luts, a.table, a.encoded, (uint32_t)a.n_bytes, a.packed, a.op, a.gaps,
                     a.out, (uint32_t)a.n_elements, (int)a.n_fb, a.cap);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

template <int kThreads, bool kChecked, bool kKindCheck>
int launch_multi(const DecodeArgs &a, int slot) {
  constexpr int kMaxSyms = kThreads * kChunkBits;
  const int mb = a.min_code_bits >= 1 && a.min_code_bits <= 16 ? a.min_code_bits : 1;
  const int run_slots = run_slots_for(mb);
  const size_t dyn =
      sizeof(uint32_t) * ((size_t)run_slots * kThreads + 2 * (size_t)stage_dwords(a.cap));
  const size_t max_dyn = sizeof(uint32_t) * ((size_t)run_slots_for(1) * kThreads +
                                             2 * (size_t)stage_dwords(kMaxSyms));
  auto kernel = decode_multi_kernel<kThreads, kChecked, kKindCheck>;
  int grid = 0;
  const int rc = persistent_grid(reinterpret_cast<const void *>(kernel), kThreads, dyn, max_dyn,
                                 slot, a.n_fb, &grid);
  if (rc != ECF8_OK) return rc;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), dyn, a.stream, a.luts,
                     a.n_luts, a.table, a.encoded, (uint32_t)a.n_bytes, a.packed, a.op, a.gaps,
                     a.out, (uint32_t)a.n_elements, (int)a.n_fb, a.cap, run_slots);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

// kind: ECF8_TABLE_DFA, ECF8_TABLE_MULTI, or ECF8_TABLE_ANY (read on the
// device: both kernels are launched, and the one the table is not for exits
// at once).
template <int kThreads>
int launch_decode(DecodeArgs a, int64_t max_block_elements, int kind, int tpb_slot) {
  constexpr int kMaxSyms = kThreads * kChunkBits;
  const int cap = (max_block_elements <= 0 || max_block_elements > kMaxSyms)
                      ? kMaxSyms
                      : (int)max_block_elements;
  a.cap = cap < 16 ? 16 : cap;
  // the clamped vector loads need 12 bitstream bytes and 8 nibble bytes
  const bool checked = a.n_bytes < 12 || a.n_elements < 16;
  const int c = checked ? 1 : 0;
  if (kind == ECF8_TABLE_DFA) {
    const int slot = 2 * tpb_slot + c;
    return checked ? launch_dfa<kThreads, true, false>(a, slot)
                   : launch_dfa<kThreads, false, false>(a, slot);
  }
  if (kind == ECF8_TABLE_MULTI) {
    const int slot = 8 + 2 * tpb_slot + c;
    return checked ? launch_multi<kThreads, true, false>(a, slot)
                   : launch_multi<kThreads, false, false>(a, slot);
  }
  const int rc = checked ? launch_dfa<kThreads, true, true>(a, 20 + 2 * tpb_slot + c)
                         : launch_dfa<kThreads, false, true>(a, 20 + 2 * tpb_slot + c);
  if (rc != ECF8_OK) return rc;
  return checked ? launch_multi<kThreads, true, true>(a, 28 + 2 * tpb_slot + c)
                 : launch_multi<kThreads, false, true>(a, 28 + 2 * tpb_slot + c);
}

template <int kThreads, bool kSelect = false>
int launch_dfa_batched(const ecf8_block_desc *descs, int count, int n_tasks, int blocks_per_task,
                       int cap, hipStream_t stream, int slot, const int *dev_counts = nullptr,
                       const int32_t *select = nullptr, int32_t *sel_counts = nullptr) {
  constexpr int kMaxSyms = kThreads * kChunkBits;
  const size_t dyn = sizeof(uint32_t) * 2 * ((size_t)stage_dwords(cap) + kSpillDwords);
  const size_t max_dyn = sizeof(uint32_t) * 2 * ((size_t)stage_dwords(kMaxSyms) + kSpillDwords);
  auto kernel = decode_dfa_batched_kernel<kThreads, kSelect>;
  int grid = 0;
  const int rc = persistent_grid(reinterpret_cast<const void *>(kernel), kThreads, dyn, max_dyn,
                                 slot, n_tasks, &grid);
  if (rc != ECF8_OK) return rc;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), dyn, stream, descs, count,
                     n_tasks, blocks_per_task, cap, dev_counts, select, sel_counts);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

int launch_dfa_bf16(const DecodeArgs &a, uint16_t *out16, const ScaleParts &parts) {
  constexpr int kThreads = 512;
  constexpr int kMaxSyms = kThreads * kChunkBits;
  const size_t dyn = sizeof(uint32_t) * 2 * ((size_t)stage_dwords(a.cap) + kSpillDwords);
  const size_t max_dyn = sizeof(uint32_t) * 2 * ((size_t)stage_dwords(kMaxSyms) + kSpillDwords);
  auto kernel = decode_dfa_bf16_kernel<kThreads>;
  int grid = 0;
  const int rc = persistent_grid(reinterpret_cast<const void *>(kernel), kThreads, dyn, max_dyn,
                                 36, a.n_fb, &grid);
  if (rc != ECF8_OK) return rc;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), dyn, a.stream, a.luts,
                     a.n_luts, a.table, a.encoded, (uint32_t)a.n_bytes, a.packed, a.op, a.gaps,
                     out16, (uint32_t)a.n_elements, (int)a.n_fb, a.cap, parts);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

}  // namespace

extern "C" int ecf8_decode_batched(const ecf8_block_desc *descs, int count, int n_tasks,
                                   int blocks_per_task, int64_t max_block_elements,
                                   int threads_per_block, void *stream) {
  if (count < 0 || n_tasks < 0 || blocks_per_task < 1) return ECF8_ERR_INVALID_ARG;
  if (count == 0 || n_tasks == 0) return ECF8_OK;
  if (!descs) return ECF8_ERR_INVALID_ARG;
  if ((uintptr_t)descs & 7) return ECF8_ERR_MISALIGNED;
  if (threads_per_block != 128 && threads_per_block != 256 && threads_per_block != 512 &&
      threads_per_block != 1024)
    return ECF8_ERR_UNSUPPORTED;
  const int64_t max_syms = (int64_t)threads_per_block * kChunkBits;
  int cap = (max_block_elements <= 0 || max_block_elements > max_syms) ? (int)max_syms
                                                                        : (int)max_block_elements;
  if (cap < 16) cap = 16;
  hipStream_t s = (hipStream_t)stream;
  switch (threads_per_block) {
    case 128:
      return launch_dfa_batched<128>(descs, count, n_tasks, blocks_per_task, cap, s, 16);
    case 256:
      return launch_dfa_batched<256>(descs, count, n_tasks, blocks_per_task, cap, s, 17);
    case 512:
      return launch_dfa_batched<512>(descs, count, n_tasks, blocks_per_task, cap, s, 18);
    default:
      return launch_dfa_batched<1024>(descs, count, n_tasks, blocks_per_task, cap, s, 19);
  }
}

extern "C" int ecf8_decode_batched_select(const ecf8_block_desc *descs, int count,
                                          const int32_t *select, ecf8_block_desc *work_descs,
                                          int32_t *work_counts, int blocks_per_task,
                                          int64_t max_block_elements, int threads_per_block,
                                          void *stream) {
  if (count < 0 || blocks_per_task < 1) return ECF8_ERR_INVALID_ARG;
  if (count == 0) return ECF8_OK;
  if (!descs || !select || !work_descs || !work_counts) return ECF8_ERR_INVALID_ARG;
  if (((uintptr_t)descs & 7) || ((uintptr_t)work_descs & 7) || ((uintptr_t)select & 3) ||
      ((uintptr_t)work_counts & 3))
    return ECF8_ERR_MISALIGNED;
  if (threads_per_block != 128 && threads_per_block != 256 && threads_per_block != 512 &&
      threads_per_block != 1024)
    return ECF8_ERR_UNSUPPORTED;
  const int64_t max_syms = (int64_t)threads_per_block * kChunkBits;
  int cap = (max_block_elements <= 0 || max_block_elements > max_syms) ? (int)max_syms
                                                                        : (int)max_block_elements;
  if (cap < 16) cap = 16;
  hipStream_t s = (hipStream_t)stream;
  // the task count is only known on the device: a full persistent grid,
  // each workgroup stops at the selected task count
  const int n_tasks_bound = INT32_MAX;
  if (count <= kLdsBlocks) {
    // one launch: every workgroup scans the flags itself (work_descs is not
    // used; workgroup 0 writes work_counts)
    switch (threads_per_block) {
      case 128:
        return launch_dfa_batched<128, true>(descs, count, n_tasks_bound, blocks_per_task, cap, s,
                                             37, nullptr, select, work_counts);
      case 256:
        return launch_dfa_batched<256, true>(descs, count, n_tasks_bound, blocks_per_task, cap, s,
                                             38, nullptr, select, work_counts);
      case 512:
        return launch_dfa_batched<512, true>(descs, count, n_tasks_bound, blocks_per_task, cap, s,
                                             39, nullptr, select, work_counts);
      default:
        return launch_dfa_batched<1024, true>(descs, count, n_tasks_bound, blocks_per_task, cap, s,
                                              40, nullptr, select, work_counts);
    }
  }
  const int64_t block_bytes = (int64_t)threads_per_block * kChunkBytes;
  hipLaunchKernelGGL(select_blocks_kernel, dim3(1), dim3(1024), 0, s, descs, count, select,
                     blocks_per_task, block_bytes, work_descs, work_counts);
  if (hipGetLastError() != hipSuccess) return ECF8_ERR_HIP;
  switch (threads_per_block) {
    case 128:
      return launch_dfa_batched<128>(work_descs, count, n_tasks_bound, blocks_per_task, cap, s, 16,
                                     work_counts);
    case 256:
      return launch_dfa_batched<256>(work_descs, count, n_tasks_bound, blocks_per_task, cap, s, 17,
                                     work_counts);
    case 512:
      return launch_dfa_batched<512>(work_descs, count, n_tasks_bound, blocks_per_task, cap, s, 18,
                                     work_counts);
    default:
      return launch_dfa_batched<1024>(work_descs, count, n_tasks_bound, blocks_per_task, cap, s,
                                      19, work_counts);
  }
}

namespace {

// ecf8_decode's checks, then (launch) its kernels.  Every argument error is
// returned before anything is launched.
int decode_checked(const uint8_t *luts, const uint8_t *encoded, const uint8_t *packed_other_4bits,
                   const uint64_t *output_positions, const uint8_t *gaps, uint8_t *outputs,
                   int n_luts, int64_t n_bytes, int64_t n_elements, int64_t max_block_elements,
                   int min_code_bits, const uint32_t *table, int table_kind,
                   int threads_per_block, int bytes_per_thread, void *stream, bool launch) {
  if (n_bytes < 0 || n_elements < 0 || (n_elements & 1)) return ECF8_ERR_INVALID_ARG;
  // the reference's positions are 32-bit (decode.cu:23-25, 151); so is this
  // kernel's index arithmetic
  if (n_bytes > INT32_MAX - 64 || n_elements > INT32_MAX - 64) return ECF8_ERR_UNSUPPORTED;
  if (bytes_per_thread != kChunkBytes) return ECF8_ERR_UNSUPPORTED;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  if (table_kind != ECF8_TABLE_MULTI && table_kind != ECF8_TABLE_DFA &&
      table_kind != ECF8_TABLE_ANY)
    return ECF8_ERR_INVALID_ARG;
  const int64_t fb_bytes = (int64_t)threads_per_block * bytes_per_thread;
  if (threads_per_block != 128 && threads_per_block != 256 && threads_per_block != 512 &&
      threads_per_block != 1024)
    return ECF8_ERR_UNSUPPORTED;
  const int64_t n_fb = (n_bytes + fb_bytes - 1) / fb_bytes;
  if (n_fb == 0) return ECF8_OK;
  if (!luts || !encoded || !output_positions || !gaps || (launch && !table) ||
      (n_elements > 0 && (!packed_other_4bits || !outputs)))
    return ECF8_ERR_INVALID_ARG;
  if (((uintptr_t)encoded & 15) || ((uintptr_t)packed_other_4bits & 7) ||
      ((uintptr_t)outputs & 15) || ((uintptr_t)table & 3) || ((uintptr_t)output_positions & 7))
    return ECF8_ERR_MISALIGNED;
  if (!launch) return ECF8_OK;
  DecodeArgs a{luts,      n_luts, table,      encoded, n_bytes, packed_other_4bits,
               output_positions, gaps, outputs, n_elements, n_fb, 0,
               min_code_bits, (hipStream_t)stream};
  switch (threads_per_block) {
    case 128:
      return launch_decode<128>(a, max_block_elements, table_kind, 0);
    case 256:
      return launch_decode<256>(a, max_block_elements, table_kind, 1);
    case 512:
      return launch_decode<512>(a, max_block_elements, table_kind, 2);
    default:
      return launch_decode<1024>(a, max_block_elements, table_kind, 3);
  }
}

}  // namespace

extern "C" int ecf8_decode(const uint8_t *luts, const uint8_t *encoded,
                           const uint8_t *packed_other_4bits, const uint64_t *output_positions,
                           const uint8_t *gaps, uint8_t *outputs, int n_luts, int64_t n_bytes,
                           int64_t n_elements, int64_t max_block_elements, int min_code_bits,
                           const uint32_t *table, int table_kind, int threads_per_block,
                           int bytes_per_thread, void *stream) {
  return decode_checked(luts, encoded, packed_other_4bits, output_positions, gaps, outputs,
                        n_luts, n_bytes, n_elements, max_block_elements, min_code_bits, table,
                        table_kind, threads_per_block, bytes_per_thread, stream, true);
}

extern "C" int ecf8_decode_bf16(const uint8_t *luts, const uint8_t *encoded,
                                const uint8_t *packed_other_4bits,
                                const uint64_t *output_positions, const uint8_t *gaps,
                                uint16_t *out_bf16, int n_luts, int64_t n_bytes,
                                int64_t n_elements, int64_t max_block_elements,
                                const uint32_t *table, int table_kind,
                                const ecf8_scaled_part *parts, int n_parts,
                                int threads_per_block, int bytes_per_thread, void *stream) {
  // ecf8_decode's checks first (the output counted as its bytes: the same
  // alignment), then this entry point's own
  const int rc = decode_checked(luts, encoded, packed_other_4bits, output_positions, gaps,
                                reinterpret_cast<uint8_t *>(out_bf16), n_luts, n_bytes,
                                n_elements, max_block_elements, 0, table, table_kind,
                                threads_per_block, bytes_per_thread, stream, false);
  if (rc != ECF8_OK) return rc;
  if (table_kind != ECF8_TABLE_DFA || threads_per_block != 512) return ECF8_ERR_UNSUPPORTED;
  if (!parts || n_parts < 1 || n_parts > ECF8_MAX_SCALED_PARTS || !table)
    return ECF8_ERR_INVALID_ARG;
  ScaleParts sp{};
  int64_t next = 0;
  for (int j = 0; j < n_parts; ++j) {
    const ecf8_scaled_part &p = parts[j];
    if (!p.scale || p.rows <= 0 || p.cols <= 0 || p.rows % 128 || p.cols % 128 ||
        p.start != next || p.rows > n_elements / p.cols)
      return ECF8_ERR_INVALID_ARG;
    if ((uintptr_t)p.scale & 3) return ECF8_ERR_MISALIGNED;
    next += p.rows * p.cols;
    const uint32_t cols = (uint32_t)p.cols;
    int sh = 0;
    while ((1ull << sh) < cols) ++sh;  // ceil(log2 cols) >= 7
    sp.p[j].start = (uint32_t)p.start;
    sp.p[j].cols = cols;
    sp.p[j].magic = (uint32_t)(((1ull << (31 + sh)) + cols - 1) / cols);
    sp.p[j].shift = (uint32_t)(sh - 1);
    sp.p[j].scale = p.scale;
  }
  if (next != n_elements) return ECF8_ERR_INVALID_ARG;
  // the kernel's clamped vector loads and its last-segment clamp
  if (n_bytes < 12 || n_elements < 16) return ECF8_ERR_UNSUPPORTED;
  sp.n = n_parts;
  constexpr int kMaxSyms = 512 * kChunkBits;
  const int64_t fb_bytes = 512 * (int64_t)kChunkBytes;
  DecodeArgs a{luts,      n_luts, table,      encoded, n_bytes, packed_other_4bits,
               output_positions, gaps, nullptr, n_elements, (n_bytes + fb_bytes - 1) / fb_bytes,
               0, 0, (hipStream_t)stream};
  const int cap = (max_block_elements <= 0 || max_block_elements > kMaxSyms)
                      ? kMaxSyms
                      : (int)max_block_elements;
  a.cap = cap < 16 ? 16 : cap;
  return launch_dfa_bf16(a, out_bf16, sp);
}

// ===========================================================================
// Allocation-free decode
// ===========================================================================
//
// The derived table of ecf8_decode_noalloc lives in `scratch`, one table per
// device, held until the process ends.  Host code never passes the array's
// name to a kernel: it is a host-side stand-in.  Its device address is taken
// once per device with hipGetSymbolAddress and kept in g_scratch.

static __device__ __align__(256) uint32_t scratch[ECF8_TABLE_BYTES / 4];

namespace {

uint32_t *g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The calling thread's current device's address of `scratch` (nullptr on a
// HIP error), looked up on the first call on that device.
uint32_t *scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch[dev] = static_cast<uint32_t *>(ptr);
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int ecf8_decode_noalloc(const uint8_t *luts, const uint8_t *encoded,
                                   const uint8_t *packed_other_4bits,
                                   const uint64_t *output_positions, const uint8_t *gaps,
                                   uint8_t *outputs, int n_luts, int64_t n_bytes,
                                   int64_t n_elements, int64_t max_block_elements,
                                   int threads_per_block, int bytes_per_thread, void *stream) {
  // Every argument error is returned before any HIP call.  One table of
  // fixed size serves every input: no size can exceed `scratch` (the LUT
  // stack is bounded by ECF8_MAX_LUTS, checked here too).
  int rc = decode_checked(luts, encoded, packed_other_4bits, output_positions, gaps, outputs,
                          n_luts, n_bytes, n_elements, max_block_elements, 0, nullptr,
                          ECF8_TABLE_ANY, threads_per_block, bytes_per_thread, stream, false);
  if (rc != ECF8_OK) return rc;
  if (n_bytes == 0) return ECF8_OK;
  if ((uintptr_t)luts & 3) return ECF8_ERR_MISALIGNED;
  uint32_t *table = scratch_on_current_device();
  if (!table) return ECF8_ERR_HIP;
  // the table builder writes every word of the table, so the previous
  // call's contents need no clearing
  rc = ecf8_build_table(luts, n_luts, ECF8_TABLE_ANY, table, nullptr, stream);
  if (rc != ECF8_OK) return rc;
  return decode_checked(luts, encoded, packed_other_4bits, output_positions, gaps, outputs,
                        n_luts, n_bytes, n_elements, max_block_elements, 0, table,
                        ECF8_TABLE_ANY, threads_per_block, bytes_per_thread, stream, true);
}
