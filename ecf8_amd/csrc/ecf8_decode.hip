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
// MI355X design (one workgroup per format-block at a time, persistent grid):
//   1. each lane loads its 8-byte chunk + 2 look-ahead bytes (coalesced
//      dwordx2 per lane) and decodes the codes it owns through a 4096-entry
//      multi-symbol table in LDS (up to 4 symbols per lookup, derived once per
//      compressed block by build_table_kernel); the exponents are packed as
//      nibbles into a lane-private LDS run;
//   2. the per-lane symbol counts are prefix-summed (wave64 shuffle scan +
//      per-wave totals in LDS), giving each lane its output offset;
//   3. each lane ORs its nibble run into a dense LDS staging array at that
//      offset (ds_or_b32, so runs sharing a dword need no ordering);
//   4. the staging array is swept in 16-element segments: 8 exponent
//      nibbles + 8 bytes of sign/mantissa nibbles become 16 FP8 bytes with
//      bitfield inserts and byte permutes, stored as one 128-bit store
//      (byte stores only on the two partial segments at the block edges).
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
constexpr int kPrivDwords = kChunkBits / 8;  // <= 64 nibbles per chunk

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
// stack, well-formed or not.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void build_table_kernel(const uint8_t *__restrict__ luts,
                                                          int n_luts,
                                                          uint32_t *__restrict__ table) {
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

template <int kThreads>
__global__ __launch_bounds__(kThreads) void decode_kernel(
    const uint8_t *__restrict__ luts, int n_luts, const uint32_t *__restrict__ table,
    const uint8_t *__restrict__ encoded, int64_t n_bytes, const uint8_t *__restrict__ packed,
    const uint64_t *__restrict__ op, const uint8_t *__restrict__ gaps,
    uint8_t *__restrict__ out, int64_t n_elements, int64_t n_fb) {
  constexpr int kWaves = kThreads / 64;
  constexpr int kMaxSyms = kThreads * kChunkBits;     // symbols a format-block can own
  constexpr int kStageDwords = kMaxSyms / 8 + 4;      // + alignment slack
  __shared__ uint32_t s_table[kTableSize];
  __shared__ uint8_t s_luts[ECF8_MAX_LUTS * 256];
  __shared__ uint32_t s_priv[kPrivDwords * kThreads];  // [dword][lane]
  __shared__ __attribute__((aligned(16))) uint32_t s_stage[kStageDwords];
  __shared__ int s_wave_sum[kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int i = tid; i < kTableSize; i += kThreads) s_table[i] = table[i];
  const int lut_bytes = n_luts * 256;
  for (int i = tid; i < ECF8_MAX_LUTS * 256; i += kThreads) s_luts[i] = i < lut_bytes ? luts[i] : 0;
  __syncthreads();
  const int len_row = (n_luts - 1) * 256;
  const uint32_t max_row = (uint32_t)(n_luts - 2);

  for (int64_t fb = blockIdx.x; fb < n_fb; fb += gridDim.x) {
    // ---- 1. load this lane's chunk (big-endian) and decode the codes it owns
    const int64_t g = fb * kThreads + tid;
    const int64_t byte0 = g * kChunkBytes;
    uint64_t hi;
    uint32_t la;
    if (byte0 + kChunkBytes + 2 <= n_bytes) {
      const uint2 d = *reinterpret_cast<const uint2 *>(encoded + byte0);
      const uint16_t l = *reinterpret_cast<const uint16_t *>(encoded + byte0 + kChunkBytes);
      hi = __builtin_bswap64(((uint64_t)d.y << 32) | d.x);
      la = __builtin_bswap16(l);
    } else {  // stream tail: bytes past n_bytes read as zero
      hi = 0;
      la = 0;
      for (int i = 0; i < kChunkBytes; ++i) {
        const int64_t j = byte0 + i;
        hi = (hi << 8) | (j < n_bytes ? encoded[j] : 0u);
      }
      for (int i = kChunkBytes; i < kChunkBytes + 2; ++i) {
        const int64_t j = byte0 + i;
        la = (la << 8) | (j < n_bytes ? encoded[j] : 0u);
      }
    }
    const uint32_t gbyte = gaps[g >> 1];
    const int gap = (g & 1) ? (gbyte & 0xF) : (gbyte >> 4);

    int p = gap;               // bit offset of the next code inside the chunk
    uint64_t buf = hi << gap;  // next code left-aligned
    uint64_t acc = 0;          // pending exponent nibbles, first in bits 0..3
    int accbits = 0, cnt = 0, j = 0;

    auto step = [&](bool tail) {
      uint32_t e = s_table[(uint32_t)(buf >> 52)];
      uint32_t len = entry_len(e);
      uint32_t syms = e & 0xFFFFu;
      uint32_t mask = entry_mask(e);
      if (len == 0) {  // code longer than 12 bits: one symbol, two-level LUT
        const uint32_t w16 = (uint32_t)(buf >> 48);
        uint32_t v = s_luts[w16 >> 8];
        if (v >= 240) {
          uint32_t row = 256 - v;
          row = row < max_row ? row : max_row;
          v = s_luts[row * 256 + (w16 & 0xFF)];
        }
        len = s_luts[len_row + v];
        syms = v & 0xF;
        mask = 1;
        if (len == 0) {  // malformed LUT: stop this chunk
          p = kChunkBits;
          return;
        }
      }
      if (tail) {  // keep only symbols that start inside this chunk
        const int rem = kChunkBits - p;
        if (rem < kWinBits) {
          const uint32_t m2 = mask & ((1u << rem) - 1);
          if (m2 != mask) {
            mask = m2;
            len = rem;
          }
        }
      }
      const uint32_t n = __builtin_popcount(mask);
      syms &= (1u << (4 * n)) - 1;
      acc |= (uint64_t)syms << accbits;
      accbits += 4 * n;
      cnt += n;
      if (accbits >= 32) {
        if (j < kPrivDwords) s_priv[j * kThreads + tid] = (uint32_t)acc;
        ++j;
        acc >>= 32;
        accbits -= 32;
      }
      p += len;
      buf <<= len;
    };

    while (p < 32) step(false);
    if (p < kChunkBits) {
      buf = ((hi << 32) | ((uint64_t)la << 16)) << (p - 32);
      while (p < kChunkBits) step(true);
    }
    if (accbits > 0 && j < kPrivDwords) s_priv[j * kThreads + tid] = (uint32_t)acc;

    // ---- 2. block-wide exclusive prefix of the per-chunk symbol counts
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d, 64);
      if (lane >= d) incl += t;
    }
    if (lane == 63) s_wave_sum[wave] = incl;

    const int64_t start = (int64_t)op[fb];
    int64_t end = (int64_t)op[fb + 1];
    if (end > n_elements) end = n_elements;
    const int64_t base = start & ~(int64_t)15;  // 16-element aligned sweep origin
    int64_t total = end - start;
    if (total < 0 || start < 0) total = 0;  // malformed positions write nothing
    if (total > kMaxSyms) total = kMaxSyms;
    const int lead = (int)(start - base);
    const int stage_nib = total > 0 ? lead + (int)total : 0;
    const int stage_dw = ((stage_nib + 15) >> 4) * 2;
    for (int i = tid; i < stage_dw; i += kThreads) s_stage[i] = 0;
    __syncthreads();

    int excl = incl - cnt;
    for (int w = 0; w < wave; ++w) excl += s_wave_sum[w];

    // ---- 3. OR this lane's nibble run into the staging array
    int c = cnt;
    if ((int64_t)excl + c > total) c = (int)(total - excl);
    if (c > 0) {
      const int nib0 = lead + excl;
      const int sh = (nib0 & 7) * 4;
      const int d0 = nib0 >> 3;
      const int ndw = (c + 7) >> 3;
      uint32_t carry = 0;
      for (int k = 0; k < ndw; ++k) {
        uint32_t v = s_priv[k * kThreads + tid];
        if (k == ndw - 1 && (c & 7)) v &= (1u << (4 * (c & 7))) - 1;
        atomicOr(&s_stage[d0 + k], (v << sh) | carry);
        carry = sh ? (v >> (32 - sh)) : 0u;
      }
      if (carry) atomicOr(&s_stage[d0 + ndw], carry);
    }
    __syncthreads();

    // ---- 4. merge with the sign/mantissa nibbles and store FP8 bytes
    const int nseg = stage_dw >> 1;
    for (int s = tid; s < nseg; s += kThreads) {
      const uint2 ev = reinterpret_cast<const uint2 *>(s_stage)[s];
      const int64_t gpos = base + 16 * (int64_t)s;
      uint2 ov;
      if (gpos + 16 <= n_elements) {
        ov = *reinterpret_cast<const uint2 *>(packed + (gpos >> 1));
      } else {
        uint32_t t[2] = {0u, 0u};
        for (int i = 0; i < 8; ++i) {
          const int64_t q = (gpos >> 1) + i;
          const uint32_t b = q < (n_elements >> 1) ? packed[q] : 0u;
          t[i >> 2] |= b << (8 * (i & 3));
        }
        ov.x = t[0];
        ov.y = t[1];
      }
      const uint2 lo = merge8(ev.x, ov.x);
      const uint2 hi8 = merge8(ev.y, ov.y);
      if (gpos >= start && gpos + 16 <= end) {
        *reinterpret_cast<uint4 *>(out + gpos) = make_uint4(lo.x, lo.y, hi8.x, hi8.y);
      } else {
        const uint32_t words[4] = {lo.x, lo.y, hi8.x, hi8.y};
        for (int i = 0; i < 16; ++i) {
          const int64_t q = gpos + i;
          if (q >= start && q < end) out[q] = (uint8_t)(words[i >> 2] >> (8 * (i & 3)));
        }
      }
    }
    __syncthreads();
  }
}

struct LaunchCache {
  int device = -1;
  int cus = 0;
  int per_cu[4] = {0, 0, 0, 0};  // occupancy for 128, 256, 512, 1024 threads
};
constexpr int kMaxDevices = 64;
LaunchCache g_cache[kMaxDevices];

template <int kThreads>
int launch_decode(const uint8_t *luts, int n_luts, const uint32_t *table, const uint8_t *encoded,
                  int64_t n_bytes, const uint8_t *packed, const uint64_t *op, const uint8_t *gaps,
                  uint8_t *out, int64_t n_elements, int64_t n_fb, hipStream_t stream, int slot) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return ECF8_ERR_HIP;
  LaunchCache &c = g_cache[dev];
  if (c.device != dev || c.cus == 0) {
    if (hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return ECF8_ERR_HIP;
    c.device = dev;
  }
  if (c.per_cu[slot] == 0) {
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_kernel<kThreads>, kThreads, 0) !=
        hipSuccess)
      return ECF8_ERR_HIP;
    c.per_cu[slot] = occ > 0 ? occ : 1;
  }
  int64_t grid = (int64_t)c.cus * c.per_cu[slot];
  if (grid > n_fb) grid = n_fb;
  hipLaunchKernelGGL(decode_kernel<kThreads>, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                     luts, n_luts, table, encoded, n_bytes, packed, op, gaps, out, n_elements,
                     n_fb);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

}  // namespace

extern "C" int ecf8_build_table(const uint8_t *luts, int n_luts, uint32_t *table, void *stream) {
  if (!luts || !table) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  hipLaunchKernelGGL(build_table_kernel, dim3(kTableSize / 256), dim3(256), 0,
                     (hipStream_t)stream, luts, n_luts, table);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

extern "C" int ecf8_decode(const uint8_t *luts, const uint8_t *encoded,
                           const uint8_t *packed_other_4bits, const uint64_t *output_positions,
                           const uint8_t *gaps, uint8_t *outputs, int n_luts, int64_t n_bytes,
                           int64_t n_elements, const uint32_t *table, int threads_per_block,
                           int bytes_per_thread, void *stream) {
  if (n_bytes < 0 || n_elements < 0 || (n_elements & 1)) return ECF8_ERR_INVALID_ARG;
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
  if (((uintptr_t)encoded & 7) || ((uintptr_t)packed_other_4bits & 7) ||
      ((uintptr_t)outputs & 15) || ((uintptr_t)table & 3) || ((uintptr_t)output_positions & 7))
    return ECF8_ERR_MISALIGNED;
  hipStream_t s = (hipStream_t)stream;
  switch (threads_per_block) {
    case 128:
      return launch_decode<128>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                output_positions, gaps, outputs, n_elements, n_fb, s, 0);
    case 256:
      return launch_decode<256>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                output_positions, gaps, outputs, n_elements, n_fb, s, 1);
    case 512:
      return launch_decode<512>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                output_positions, gaps, outputs, n_elements, n_fb, s, 2);
    default:
      return launch_decode<1024>(luts, n_luts, table, encoded, n_bytes, packed_other_4bits,
                                 output_positions, gaps, outputs, n_elements, n_fb, s, 3);
  }
}
