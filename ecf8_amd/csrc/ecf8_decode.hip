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
// MI355X design (one workgroup per format-block at a time, persistent grid,
// the next block's bitstream prefetched while the current one decodes):
//   1. each lane takes one chunk (one 128-bit load: chunk + look-ahead) and
//      decodes the codes it owns through a 4096-entry multi-symbol table in
//      LDS (up to 4 symbols per lookup, derived once per compressed block by
//      build_table_kernel); exponents are ORed as nibbles into a lane-private
//      LDS run (ds_or_b32, no per-symbol bookkeeping branches);
//   2. the per-chunk symbol counts are prefix-summed (wave64 DPP scan +
//      per-wave totals in LDS), giving each lane its output offset;
//   3. each lane ORs its nibble run into a dense LDS staging buffer at that
//      offset (double-buffered across blocks, sized from the largest block
//      of the tensor like the reference's shared_mem_size);
//   4. the staging buffer is swept in 16-element segments: 8 exponent
//      nibbles + 8 bytes of sign/mantissa nibbles (prefetched at block
//      start) become 16 FP8 bytes with bitfield inserts and byte permutes,
//      stored as one 128-bit store (byte stores only on the two partial
//      segments at the block edges).
// All work is integer VALU/LDS; the HBM traffic is the compressed bytes read
// once and the FP8 bytes written once.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ecf8.h"

namespace {

constexpr int kWinBits = 12;                 // multi-symbol table index width
constexpr int kTableSize = 1 << kWinBits;    // 4096 entries, u32 each
constexpr int kMaxSymsPerEntry = 4;
constexpr int kChunkBytes = 8;               // bytes_per_thread of the format
constexpr int kChunkBits = 8 * kChunkBytes;

// Table entry layout:
//   bits  0..15  up to 4 exponents, first decoded in bits 0..3
//   bits 16..27  start mask: bit j set iff one of those symbols starts at
//                window offset j (so popcount = number of symbols)
//   bits 28..31  total code length of those symbols (0 = no symbol fully
//                determined by the 12 window bits; decode one symbol with
//                the two-level LUT instead)
__host__ __device__ constexpr uint32_t entry_len(uint32_t e) { return e >> 28; }
__host__ __device__ constexpr uint32_t entry_mask(uint32_t e) { return (e >> 16) & 0xFFFu; }

// ---------------------------------------------------------------------------
// Table builder: one thread per 12-bit window value.  Symbols are accepted
// only while the reference rule's result provably does not depend on the
// bits after the window (every LUT entry the unknown bits could select holds
// the same value), so the table reproduces the rule exactly for any LUT
// stack, well-formed or not.  The LUT stack (at most 18 x 256 bytes) is
// staged in LDS first: the constancy checks read up to 128 entries per step.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void build_table_kernel(const uint8_t *__restrict__ g_luts,
                                                          int n_luts,
                                                          uint32_t *__restrict__ table) {
  __shared__ uint32_t s_lut_words[ECF8_MAX_LUTS * 64];
  const int n_words = n_luts * 64;
  for (int i = threadIdx.x; i < n_words; i += blockDim.x)
    s_lut_words[i] = reinterpret_cast<const uint32_t *>(g_luts)[i];
  __syncthreads();
  const uint8_t *const luts = reinterpret_cast<const uint8_t *>(s_lut_words);
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= kTableSize) return;
  const uint8_t *len_row = luts + 256 * (n_luts - 1);
  uint32_t syms = 0, mask = 0;
  int n = 0, off = 0;
  while (n < kMaxSymsPerEntry && off < kWinBits) {
    const int known = kWinBits - off;  // window bits from this symbol's start
    // first level: the 8 bits at the symbol start
    const int kb = known < 8 ? known : 8;
    const int idx = ((w >> (known - kb)) & ((1 << kb) - 1)) << (8 - kb);
    const int span = 1 << (8 - kb);
    int v = luts[idx];
    bool fixed = true;
    for (int x = 1; x < span; ++x) fixed &= luts[idx + x] == v;
    if (!fixed) break;
    if (v >= 240) {
      const int row = 256 - v;
      if (row > n_luts - 2) break;
      const int known2 = known - 8;  // bits of the second byte inside the window
      const int kb2 = known2 <= 0 ? 0 : (known2 < 8 ? known2 : 8);
      const int idx2 = kb2 ? ((w >> (known2 - kb2)) & ((1 << kb2) - 1)) << (8 - kb2) : 0;
      const int span2 = 1 << (8 - kb2);
      const uint8_t *r = luts + 256 * row;
      v = r[idx2];
      for (int x = 1; x < span2; ++x) fixed &= r[idx2 + x] == v;
      if (!fixed) break;
    }
    const int len = len_row[v];
    if (len == 0 || len > known || v > 15) break;
    syms |= (uint32_t)v << (4 * n);
    mask |= 1u << off;
    ++n;
    off += len;
  }
  table[w] = n ? (syms | (mask << 16) | ((uint32_t)off << 28)) : 0u;
}

__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
  return (a & m) | (b & ~m);
}

// 8 FP8 bytes from 8 exponent nibbles (E, element k in bits 4k..4k+3) and
// 4 packed sign/mantissa bytes (O, byte j = o_{2j} << 4 | o_{2j+1}).
__device__ __forceinline__ uint2 merge8(uint32_t e, uint32_t o) {
  // even elements 2j: sign = O_j bit 7, exponent = E_j low nibble,
  // mantissa = O_j bits 4..6
  const uint32_t h = bfi(0x80808080u, o, bfi(0x78787878u, e << 3, o >> 4));
  // odd elements 2j+1: sign = O_j bit 3, exponent = E_j high nibble,
  // mantissa = O_j bits 0..2
  const uint32_t l = bfi(0x80808080u, o << 4, bfi(0x78787878u, e >> 1, o));
  uint2 r;
  r.x = __builtin_amdgcn_perm(h, l, 0x01050004u);  // h0 l0 h1 l1
  r.y = __builtin_amdgcn_perm(h, l, 0x03070206u);  // h2 l2 h3 l3
  return r;
}

// Inclusive prefix sum over a wave64 with DPP row shifts and row
// broadcasts (six VALU ops, no LDS round trip).
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

// ---------------------------------------------------------------------------
// Decoder: one workgroup of T threads per format-block of T chunks at a time
// (persistent grid; the next block's bitstream is fetched while the current
// one decodes), one chunk per lane.  Index arithmetic is 32-bit (the
// format's positions are < 2^31).
// ---------------------------------------------------------------------------

typedef uint32_t u32x3_a8 __attribute__((ext_vector_type(3), aligned(8)));

// A chunk as fetched: 12 raw bytes from the chunk start (8 chunk bytes, 2
// look-ahead bytes, 2 unused; little-endian dwords) and the byte holding its
// gap nibble.  Fetching never waits; the bytes are interpreted a whole
// decode phase later.
struct RawChunk {
  u32x3_a8 v;
  uint32_t gap_byte;
};

// The chunk as a big-endian bit string (hi), its two look-ahead bytes (la)
// and its gap.
struct Chunk {
  uint64_t hi;
  uint32_t la;
  uint32_t gap;
};

// Unconditional 96-bit load of chunk g, the address clamped to the last
// full 12-byte window so it stays in bounds; lanes near the stream end are
// re-read byte-wise in finish_chunk.
__device__ __forceinline__ RawChunk fetch_chunk(const uint8_t *__restrict__ encoded, uint32_t last12,
                                                const uint8_t *__restrict__ gaps, uint32_t g) {
  RawChunk r;
  const uint32_t b = g * kChunkBytes;
  r.v = *reinterpret_cast<const u32x3_a8 *>(encoded + (b < last12 ? b : last12));
  r.gap_byte = gaps[g >> 1];
  return r;
}

__device__ __forceinline__ Chunk finish_chunk(const RawChunk &r, const uint8_t *__restrict__ encoded,
                                              uint32_t n_bytes, uint32_t g, bool vector_ok) {
  Chunk c;
  const uint32_t b = g * kChunkBytes;
  if (vector_ok && b + 12 <= n_bytes) {
    c.hi = __builtin_bswap64(((uint64_t)r.v.y << 32) | r.v.x);
    c.la = ((r.v.z & 0xFFu) << 8) | ((r.v.z >> 8) & 0xFFu);
  } else {  // stream tail: bytes past n_bytes read as zero
    uint64_t hi = 0;
    uint32_t la = 0;
    for (int i = 0; i < kChunkBytes; ++i) {
      const uint32_t j = b + i;
      hi = (hi << 8) | (j < n_bytes ? encoded[j] : 0u);
    }
    for (int i = kChunkBytes; i < kChunkBytes + 2; ++i) {
      const uint32_t j = b + i;
      la = (la << 8) | (j < n_bytes ? encoded[j] : 0u);
    }
    c.hi = hi;
    c.la = la;
  }
  c.gap = (g & 1) ? (r.gap_byte & 0xFu) : (r.gap_byte >> 4);
  return c;
}

// Bits [p, p+16) of the 80-bit string hi:la (chunk + look-ahead), p < 64.
__device__ __forceinline__ uint32_t window16(uint64_t hi, uint32_t la, int p) {
  const uint64_t w = p < 48 ? (hi << p) : (((hi << 32) | ((uint64_t)la << 16)) << (p - 32));
  return (uint32_t)(w >> 48);
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

// Dwords of a lane's nibble run: room for every symbol a chunk can own when
// no code is shorter than min_bits, plus the spill dword of the last 64-bit OR.
__host__ __device__ constexpr int run_slots_for(int min_bits) {
  return ((kChunkBits + min_bits - 1) / min_bits + 7) / 8 + 1;
}
constexpr int kZeroEntry = kTableSize;          // all-zero table entry: a lookup that does nothing

// kChecked: tensors too small for the clamped vector loads (fewer than 12
// bitstream bytes or 16 elements) use byte-wise loads throughout.
//
// SGPRs are capped at 80: measured on MI355X, at 99 SGPRs only 7 waves of
// 8 per SIMD fit (3 workgroups of 512 per CU instead of 4); the few spills
// the cap causes go to VGPR lanes.
template <int kThreads, bool kChecked>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_num_sgpr(80))) void decode_kernel(
    const uint8_t *__restrict__ luts, int n_luts, const uint32_t *__restrict__ table,
    const uint8_t *__restrict__ encoded, uint32_t n_bytes, const uint8_t *__restrict__ packed,
    const uint64_t *__restrict__ op, const uint8_t *__restrict__ gaps,
    uint8_t *__restrict__ out, uint32_t n_elements, int n_fb, int stage_cap, int run_slots) {
  constexpr int kWaves = kThreads / 64;
  // dynamic LDS: [run_slots][kThreads] nibble runs, then 2 staging buffers
  extern __shared__ __attribute__((aligned(16))) uint32_t s_dyn[];
  __shared__ uint32_t s_table[kTableSize + 1];
  __shared__ int s_wave_sum[kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int stage_dw = stage_dwords(stage_cap);
  uint32_t *const s_stage = s_dyn + run_slots * kThreads;
  uint32_t *const run = s_dyn + tid;  // slot k at run[k * kThreads]
  const int max_slot = run_slots - 2;  // last slot a 64-bit OR may start in

  for (int i = tid; i <= kTableSize; i += kThreads) s_table[i] = i < kTableSize ? table[i] : 0u;
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
  // Positions are below 2^31 (checked on the host), so only the low dword of
  // each little-endian u64 is loaded: a dead high half would be reused as a
  // temporary and force an early wait on every load in flight.
  const uint32_t *const op32 = reinterpret_cast<const uint32_t *>(op);
  // this block's output range [op_lo, op_hi), wave-uniform.  Positions are
  // always read (readlane waits on the vector load) before the block's
  // stores are issued: the memory counter also counts stores, so a later
  // wait would drain them too.
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
    // prefetch target: the next block, or this one again after the last (in
    // bounds, discarded) so no load or wait depends on a branch
    const int fb_pf = fb_next < n_fb ? fb_next : fb;

    // ---- this block's output range; prefetch its sign/mantissa bytes
    const uint32_t start = op_lo;
    uint32_t end = op_hi;
    if (end > n_elements) end = n_elements;
    int total = (int)end - (int)start;
    if (total < 0 || start > n_elements) total = 0;  // malformed positions write nothing
    if (total > stage_cap) total = stage_cap;
    const uint32_t base = start & ~15u;  // 16-element aligned sweep origin
    const int lead = (int)(start - base);
    const int stage_nib = total > 0 ? lead + total : 0;
    const int seg_dw = ((stage_nib + 15) >> 4) * 2;
    const int nseg = seg_dw >> 1;
    uint2 pre0 = make_uint2(0, 0), pre1 = make_uint2(0, 0);
    if (!kChecked) {
      // segments past nseg re-read the last one (no extra HBM traffic)
      const int last_seg = nseg > 0 ? nseg - 1 : 0;
      uint32_t q0 = (base >> 1) + 8u * (uint32_t)min(tid, last_seg);
      uint32_t q1 = (base >> 1) + 8u * (uint32_t)min(tid + kThreads, last_seg);
      pre0 = *reinterpret_cast<const uint2 *>(packed + (q0 < last8 ? q0 : last8));
      pre1 = *reinterpret_cast<const uint2 *>(packed + (q1 < last8 ? q1 : last8));
    }

    // ---- prefetch the next block's chunk and positions (vector loads, so
    // the LDS waits of the decode below never wait on them)
    const RawChunk nxt_raw = fetch(fb_pf);
    const uint32_t nopv = op32[2 * (fb_pf + (lane & 1))];

    // ---- 1. decode the codes this lane's chunk owns into its nibble run
    for (int k = 0; k < run_slots; ++k) run[k * kThreads] = 0u;
    const int zero4 = (seg_dw + 3) >> 2;
    for (int i = tid; i < zero4; i += kThreads)
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
    // zero entry, which changes nothing
    bool act = e != 0 && p < 53;
    while (__builtin_amdgcn_ballot_w64(act)) {
      e = s_table[act ? (uint32_t)(buf >> 52) : (uint32_t)kZeroEntry];
      const uint32_t len = entry_len(e);
      emit(e, __builtin_popcount(entry_mask(e)));
      p += (int)len;
      buf <<= len;
      act = act && e != 0 && p < 53;
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
        act = act && e != 0 && p < kChunkBits;
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
    int excl = incl - cnt;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      if (w < wave) excl += s_wave_sum[w];

    // ---- 3. OR this lane's nibble run into the staging buffer
    int c = cnt;
    if (excl + c > total) c = total - excl;
    if (c > 0) {
      const int nib0 = lead + excl;
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

    // the next block's chunk and positions, fetched a whole decode phase ago
    const Chunk nxt = finish_chunk(nxt_raw, encoded, n_bytes, (uint32_t)fb_pf * kThreads + tid,
                                   !kChecked);
    const uint32_t nop_lo = __builtin_amdgcn_readlane(nopv, 0);
    const uint32_t nop_hi = __builtin_amdgcn_readlane(nopv, 1);

    // ---- 4. merge with the sign/mantissa nibbles and store FP8 bytes
    for (int s = tid, k = 0; s < nseg; s += kThreads, ++k) {
      const uint2 ev = reinterpret_cast<const uint2 *>(stage)[s];
      const uint32_t gpos = base + 16u * (uint32_t)s;
      uint2 ov = k == 0 ? pre0 : pre1;
      if (kChecked || k > 1 || gpos + 16 > n_elements)
        ov = load_nibbles_checked(packed, n_elements, gpos);
      const uint2 lo = merge8(ev.x, ov.x);
      const uint2 hi8 = merge8(ev.y, ov.y);
      if (gpos >= start && gpos + 16 <= end) {
        *reinterpret_cast<uint4 *>(out + gpos) = make_uint4(lo.x, lo.y, hi8.x, hi8.y);
      } else {
        const uint32_t words[4] = {lo.x, lo.y, hi8.x, hi8.y};
        for (int i = 0; i < 16; ++i) {
          const uint32_t q = gpos + i;
          if (q >= start && q < end) out[q] = (uint8_t)(words[i >> 2] >> (8 * (i & 3)));
        }
      }
    }
    // the next iteration writes the other staging buffer; its barrier after
    // the scan orders this sweep before any reuse of this one
    if (fb_next >= n_fb) break;
    fb = fb_next;
    cur = nxt;
    op_lo = nop_lo;
    op_hi = nop_hi;
  }
}

struct LaunchCache {
  int device = -1;
  int cus = 0;
  size_t occ_dyn[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // dynamic LDS of occ below
  int occ[8] = {0, 0, 0, 0, 0, 0, 0, 0};         // per (threads slot, checked) variant
  bool attr_set[8] = {false, false, false, false, false, false, false, false};
};
constexpr int kMaxDevices = 64;
LaunchCache g_cache[kMaxDevices];

template <int kThreads, bool kChecked>
int launch_variant(const uint8_t *luts, int n_luts, const uint32_t *table, const uint8_t *encoded,
                   int64_t n_bytes, const uint8_t *packed, const uint64_t *op, const uint8_t *gaps,
                   uint8_t *out, int64_t n_elements, int64_t n_fb, int cap, int run_slots,
                   hipStream_t stream, int slot) {
  constexpr int kMaxSyms = kThreads * kChunkBits;
  const size_t dyn =
      sizeof(uint32_t) * ((size_t)run_slots * kThreads + 2 * (size_t)stage_dwords(cap));
  auto kernel = decode_kernel<kThreads, kChecked>;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return ECF8_ERR_HIP;
  LaunchCache &c = g_cache[dev];
  if (c.device != dev || c.cus == 0) {
    if (hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return ECF8_ERR_HIP;
    c.device = dev;
  }
  if (!c.attr_set[slot]) {
    const size_t max_dyn = sizeof(uint32_t) * ((size_t)run_slots_for(1) * kThreads +
                                               2 * (size_t)stage_dwords(kMaxSyms));
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_dyn) != hipSuccess)
      return ECF8_ERR_HIP;
    c.attr_set[slot] = true;
  }
  if (c.occ_dyn[slot] != dyn) {
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, kThreads, dyn) != hipSuccess)
      return ECF8_ERR_HIP;
    c.occ[slot] = occ > 0 ? occ : 1;
    c.occ_dyn[slot] = dyn;
  }
  int64_t grid = (int64_t)c.cus * c.occ[slot];
  if (grid > n_fb) grid = n_fb;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), dyn, stream, luts, n_luts,
                     table, encoded, (uint32_t)n_bytes, packed, op, gaps, out,
                     (uint32_t)n_elements, (int)n_fb, cap, run_slots);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

template <int kThreads>
int launch_decode(const uint8_t *luts, int n_luts, const uint32_t *table, const uint8_t *encoded,
                  int64_t n_bytes, const uint8_t *packed, const uint64_t *op, const uint8_t *gaps,
                  uint8_t *out, int64_t n_elements, int64_t n_fb, int64_t max_block_elements,
                  int min_code_bits, hipStream_t stream, int slot) {
  constexpr int kMaxSyms = kThreads * kChunkBits;
  int cap = (max_block_elements <= 0 || max_block_elements > kMaxSyms) ? kMaxSyms
                                                                        : (int)max_block_elements;
  if (cap < 16) cap = 16;
  const int run_slots = run_slots_for(min_code_bits >= 1 && min_code_bits <= 16 ? min_code_bits : 1);
  // the clamped vector loads need 12 bitstream bytes and 8 nibble bytes
  if (n_bytes < 12 || n_elements < 16)
    return launch_variant<kThreads, true>(luts, n_luts, table, encoded, n_bytes, packed, op, gaps,
                                          out, n_elements, n_fb, cap, run_slots, stream,
                                          2 * slot + 1);
  return launch_variant<kThreads, false>(luts, n_luts, table, encoded, n_bytes, packed, op, gaps,
                                         out, n_elements, n_fb, cap, run_slots, stream, 2 * slot);
}

}  // namespace

extern "C" int ecf8_build_table(const uint8_t *luts, int n_luts, uint32_t *table, void *stream) {
  if (!luts || !table) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  if (((uintptr_t)luts & 3) || ((uintptr_t)table & 3)) return ECF8_ERR_MISALIGNED;
  hipLaunchKernelGGL(build_table_kernel, dim3(kTableSize / 256), dim3(256), 0,
                     (hipStream_t)stream, luts, n_luts, table);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

extern "C" int ecf8_decode(const uint8_t *luts, const uint8_t *encoded,
                           const uint8_t *packed_other_4bits, const uint64_t *output_positions,
                           const uint8_t *gaps, uint8_t *outputs, int n_luts, int64_t n_bytes,
                           int64_t n_elements, int64_t max_block_elements, int min_code_bits,
                           const uint32_t *table, int threads_per_block, int bytes_per_thread,
                           void *stream) {
  if (n_bytes < 0 || n_elements < 0 || (n_elements & 1)) return ECF8_ERR_INVALID_ARG;
  // the reference's positions are 32-bit (decode.cu:23-25, 151); so is this
  // kernel's index arithmetic
  if (n_bytes > INT32_MAX - 64 || n_elements > INT32_MAX - 64) return ECF8_ERR_UNSUPPORTED;
  if (bytes_per_thread != kChunkBytes) return ECF8_ERR_UNSUPPORTED;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  const int64_t fb_bytes = (int64_t)threads_per_block * bytes_per_thread;
  if (threads_per_block != 128 && threads_per_block != 256 && threads_per_block != 512 &&
      threads_per_block != 1024)
    return ECF8_ERR_UNSUPPORTED;
  const int64_t n_fb = (n_bytes + fb_bytes - 1) / fb_bytes;
  if (n_fb == 0) return ECF8_OK;
  if (!luts || !encoded || !output_positions || !gaps || !table ||
      (n_elements > 0 && (!packed_other_4bits || !outputs)))
    return ECF8_ERR_INVALID_ARG;
  if (((uintptr_t)encoded & 15) || ((uintptr_t)packed_other_4bits & 7) ||
      ((uintptr_t)outputs & 15) || ((uintptr_t)table & 3) || ((uintptr_t)output_positions & 7))
    return ECF8_ERR_MISALIGNED;
  hipStream_t s = (hipStream_t)stream;
  switch (threads_per_block) {
    case 128:
      return launch_decode<128>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                output_positions, gaps, outputs, n_elements, n_fb, max_block_elements,
                                min_code_bits, s, 0);
    case 256:
      return launch_decode<256>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                output_positions, gaps, outputs, n_elements, n_fb, max_block_elements,
                                min_code_bits, s, 1);
    case 512:
      return launch_decode<512>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                output_positions, gaps, outputs, n_elements, n_fb, max_block_elements,
                                min_code_bits, s, 2);
    default:
      return launch_decode<1024>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                 output_positions, gaps, outputs, n_elements, n_fb, max_block_elements,
                                min_code_bits, s, 3);
  }
}
