// Kernels over the tiled execution layout ECF8-T (ecf8_tile_layout.h).
//
// tile_linear16_kernel: the small-M (M <= 16, a decode step) block-scaled
//   FP8 linear with its weight operands decoded on the fly: each wave
//   decodes one 2048-symbol segment -- the B operands of its four MFMAs of
//   one 128-column group -- into a wave-private LDS staging area, reads its
//   lane's 32 exponents back, merges them with the sign/mantissa nibbles and
//   runs v_mfma_f32_16x16x32_fp8_fp8.  No FP8 weight reaches HBM.  The K
//   groups go to the waves, the products are scaled and summed, and the
//   waves' partial sums are reduced, in exactly the order of the FP8
//   linear (fp8_linear16_kernel / fp8_linear16p_kernel in ecf8_llm.hip) with
//   the same wave count, so both give bit-identical outputs.
// tile_decode_kernel: the same per-wave decode, written out as row-major
//   FP8 bytes (the prompt's large-M linears read those).
//
// A wave's decode needs no workgroup barrier: its 64 lanes decode the
// segment's 12-byte chunks with the byte automaton (12 lookups, plus the
// code open at the chunk end), a wave64 prefix sum places each lane's
// symbols, and the lanes OR them into the wave's staging area.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "ecf8.h"
#include "ecf8_dev.h"
#include "ecf8_layout.h"
#include "ecf8_llm.h"
#include "ecf8_tile.h"
#include "ecf8_tile_layout.h"

namespace {

using namespace ecf8;
using namespace ecf8::dev;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kGroup = 128;
constexpr int kStageDw = kTileSegSymbols / 8;           // 256 dwords of nibbles
constexpr int kWaveStageDw = kStageDw + 8;              // + spill for symbols past 2048
// outputs of a tiled kernel handed a table that is not an automaton
constexpr uint16_t kBf16Nan = 0x7FC0;
constexpr uint32_t kFp8Nan4 = 0x7F7F7F7Fu;  // four e4m3fn NaNs
static_assert(4 * 64 <= kWaveStageDw, "a wave's staging area holds its 4x64 partial sums");

// One weight operand of a (possibly fused) tiled linear.
struct TileOperand {
  const uint8_t *stream;
  const uint32_t *seg_off;
  const uint32_t *gaps;
  const uint8_t *other;
  const float *ws;  // weight_scale_inv [n/128, K/128]
};

struct TileSegs {
  TileOperand op[ECF8_LINEAR_MAX_SEGS];
  int n_end[ECF8_LINEAR_MAX_SEGS];  // cumulative output columns
  int col[ECF8_LINEAR_MAX_SEGS];    // first output column
  int count;
};

__device__ __forceinline__ float bf16_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// Raw buffer resources: a wave-uniform base in scalar registers and a
// 32-bit lane offset per load (instead of a 64-bit address per lane and
// load), extent unbounded (the offsets come from the layout's own
// indices).
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc_at(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, -1, 0x00020000);
}

// fp32 -> bf16, round to nearest even (as the FP8 linear does)
__device__ __forceinline__ uint32_t f32_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// 8 FP8 bytes -- operand elements 8r..8r+7 of a lane, as two dwords of 4
// -- from its staged exponent dword E (elements 0..3 in the even nibbles,
// 4..7 in the odd ones) and nibble dword O, whose byte q holds element q's
// mantissa (bits 0..2) and sign (bit 7) where its FP8 byte has them, and
// element q + 4's mantissa in bits 4..6 and sign one byte up, in bit 3 of
// byte (q + 1) % 4: rotated right by 4 bits, O holds elements 4..7 in
// place.  Five VALU ops per 8 bytes; the run order of the layout needs no
// byte interleave.
__device__ __forceinline__ uint2 merge8_runs(uint32_t e, uint32_t o) {
  uint2 r;
  r.x = bfi<0x78787878u>(e << 3, o);
  r.y = bfi<0x78787878u>(e >> 1, __builtin_amdgcn_alignbit(o, o, 4u));
  return r;
}

// A segment's code window: 16 bytes from the lane's chunk start (12 + look-
// ahead) and the gap word holding the lane's nibble.
struct SegLoad {
  uint32_t d0, d1, d2, d3;
  uint32_t gapw;
  int n_chunks;  // wave-uniform
};

// The window of segment s, whose codes occupy bytes [off, end) of the stream.
__device__ __forceinline__ SegLoad seg_window(const TileOperand &t, uint32_t s, uint32_t off,
                                              uint32_t end, int lane) {
  SegLoad r;
  r.n_chunks = (int)((end - off + kTileChunkBytes - 1) / kTileChunkBytes);
  // lanes past the segment's chunks re-read its first one (in bounds; unused)
  const uint32_t b = lane < r.n_chunks ? (uint32_t)(kTileChunkBytes * lane) : 0u;
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc_at(t.stream + off), b, 0, 0);
  r.d0 = v.x;
  r.d1 = v.y;
  r.d2 = v.z;
  r.d3 = v.w;
  r.gapw = __builtin_amdgcn_raw_buffer_load_b32(rsrc_at(t.gaps + (size_t)s * kTileGapWords),
                                                4u * (uint32_t)(lane >> 3), 0, 0);
  return r;
}

// The lane's 32 sign/mantissa nibbles of segment s (read once: streamed).
__device__ __forceinline__ u32x4 seg_other(const TileOperand &t, uint32_t s, int lane) {
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc_at(t.other + (size_t)s * kTileOtherBytes),
                                               16u * (uint32_t)lane, 0, 2 /* nt */);
}

// Byte i (0..15) of the lane's chunk window, shifted into a table offset
// (byte << 2), from its little-endian dwords (i a constant after
// unrolling): one SDWA shift that selects the byte.
__device__ __forceinline__ uint32_t byte_off(const SegLoad &c, int i) {
  const uint32_t d = i < 4 ? c.d0 : i < 8 ? c.d1 : i < 12 ? c.d2 : c.d3;
  uint32_t r;
  switch (i & 3) {
    case 0:
      asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
          "src1_sel:BYTE_0" : "=v"(r) : "v"(d));
      break;
    case 1:
      asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
          "src1_sel:BYTE_1" : "=v"(r) : "v"(d));
      break;
    case 2:
      asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
          "src1_sel:BYTE_2" : "=v"(r) : "v"(d));
      break;
    default:
      asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
          "src1_sel:BYTE_3" : "=v"(r) : "v"(d));
      break;
  }
  return r;
}

// The automaton entry after `e` on the byte at table offset `off`: the
// entry's next row (bits 10..14) and the offset (bits 2..9) merged by one
// v_bfi_b32 -- the only VALU op between two lookups of a walk.
__device__ __forceinline__ uint32_t dfa_next(const uint32_t *s_dfa, uint32_t e, uint32_t off) {
  return dfa_at(s_dfa, bfi<kDfaRowMask>(e, off));
}

// Decode N segments at once, segment j into the staging area stage + j *
// kWaveStageDw, and return each lane's 32 exponents of each (symbol 32 lane
// + k in bits 4(k%8).. of component k/8).  The N automaton walks are
// independent chains of LDS lookups: issued interleaved, each one's round
// trips hide the other's.  The staging areas are all zero on entry and on
// return (each lane clears the four dwords it read; symbols past 2048 go to
// the spill dwords, which are never read).
template <int N>
__device__ __forceinline__ void decode_segments(const SegLoad (&c)[N], const uint32_t *s_dfa,
                                                uint32_t *stage, int lane, uint4 (&ex)[N]) {
  uint32_t e[N][12];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const uint32_t gap = (c[j].gapw >> (4 * (lane & 7))) & 0xFu;
    // start row: skip `gap` bits of byte 0, or (gap >= 8) take the entry
    // that skips byte 0 into row gap - 8 (both computed, one selected)
    const uint32_t a_in = (gap << 10) | byte_off(c[j], 0);
    const uint32_t a_skip = (uint32_t)(kDfaSkipByte * 4) + ((gap - 8) << 2);
    e[j][0] = dfa_at(s_dfa, gap < 8 ? a_in : a_skip);
  }
  // each pair of entries, once both are in: its symbols (entry b's after
  // entry a's count) and its count field sum, so the pair's two entries
  // need not stay live until the staging
  uint32_t sy[N][6], s2[N][6];
  auto pair = [&](int j, int i) {
    const uint32_t ea = e[j][2 * i], eb = e[j][2 * i + 1];
    uint32_t t;
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
        "src1_sel:WORD_1"
        : "=v"(t) : "v"(ea), "v"(eb));
    asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
        "src1_sel:WORD_1"
        : "=v"(sy[j][i]) : "v"(t), "v"(ea));
    s2[j][i] = ea + eb;
  };
#pragma unroll
  for (int i = 1; i < 12; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j) {
      e[j][i] = dfa_next(s_dfa, e[j][i - 1], byte_off(c[j], i));
      if (i & 1) pair(j, i >> 1);
    }
  // a code still open at the chunk's end started in it: the chunk owns it,
  // and its symbol is the first one completed in look-ahead byte 12 or 13
  uint32_t e12[N];
  bool open[N], late = false;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const uint32_t row11 = e[j][11] & kDfaRowMask;
    open[j] = row11 >= ((uint32_t)kDfaFirstPendingRow << 10);
    e12[j] = dfa_next(s_dfa, e[j][11], byte_off(c[j], 12));
    late = late || (open[j] && (e12[j] & 0xFFu) == 0);
  }
  if (__builtin_amdgcn_ballot_w64(late)) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const uint32_t e13 = dfa_next(s_dfa, e12[j], byte_off(c[j], 13));
      if ((e12[j] & 0xFFu) == 0) e12[j] = e13;
    }
  }
  int cnt4[N];
  uint32_t et[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    et[j] = open[j] ? ((e12[j] & 0xF0000u) | 4u) : 0u;
    // the count fields (bits 0..7, at most 16 each, bits 8..9 clear) summed
    // by adding whole entries: 13 of them stay below 256, so the low byte
    // of the sum is exact
    const uint32_t sum = s2[j][0] + s2[j][1] + s2[j][2] + s2[j][3] + s2[j][4] + s2[j][5] + et[j];
    cnt4[j] = lane < c[j].n_chunks ? (int)(sum & 0xFFu) : 0;
  }
  int incl[N];
#pragma unroll
  for (int j = 0; j < N; ++j) incl[j] = wave_inclusive_scan(cnt4[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    // the staging area's LDS byte address x 8, plus the lane's first bit:
    // a bit address, whose dword is (bit >> 3) & ~3 (the area is dword
    // aligned).  A start past the real symbols (garbage decoded from the
    // bytes after the segment) is clamped to the spill dwords' start; 12
    // entries of <= 16 bits plus 4 stay within them
    typedef __attribute__((address_space(3))) uint32_t LdsU32;
    const uint32_t st_bits =
        (uint32_t)(uintptr_t)(LdsU32 *)(stage + j * kWaveStageDw) << 3;
    uint32_t bit = st_bits + min((uint32_t)(incl[j] - cnt4[j]), (uint32_t)kStageDw << 5);
    auto put = [&](uint32_t syms, uint32_t n4) {
      const uint64_t v = (uint64_t)syms << (bit & 31u);
      uint32_t *const q = (uint32_t *)(LdsU32 *)(uintptr_t)((bit >> 3) & ~3u);
      atomicOr(q, (uint32_t)v);
      atomicOr(q + 1, (uint32_t)(v >> 32));
      bit += n4;
    };
    if (lane < c[j].n_chunks) {
#pragma unroll
      for (int i = 0; i < 6; ++i) put(sy[j][i], s2[j][i] & 0xFFu);
      put(et[j] >> 16, 0u);
    }
  }
  // the wave's own ORs complete before its lanes read the staged symbols
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < N; ++j) {
    uint4 *const mine = reinterpret_cast<uint4 *>(stage + j * kWaveStageDw) + lane;
    ex[j] = *mine;
    *mine = make_uint4(0u, 0u, 0u, 0u);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ uint4 decode_segment(const SegLoad &c, const uint32_t *s_dfa,
                                                uint32_t *stage, int lane) {
  const SegLoad cs[1] = {c};
  uint4 ex[1];
  decode_segments<1>(cs, s_dfa, stage, lane, ex);
  return ex[0];
}

// Operand address of the panel `panel` (16 output columns) of the fused
// segments: its operand, the panel index inside it, its output column.
__device__ __forceinline__ void panel_of(const TileSegs &segs, int panel, TileOperand &op,
                                         int &p, int &col) {
  int n0 = panel * 16, start = 0, k = 0;
#pragma unroll
  for (int s = 1; s < ECF8_LINEAR_MAX_SEGS; ++s)
    if (s < segs.count && n0 >= segs.n_end[s - 1]) {
      k = s;
      start = segs.n_end[s - 1];
    }
  op = segs.op[k];
  col = segs.col[k];
  p = (n0 - start) / 16;
}

// The panels of a dense linear's workgroup walk: its fused operands, as one
// run of panels (a wave's steps may cross from one operand to the next).
struct DenseWalk {
  const TileSegs *segs;  // the kernel argument itself: indexed in place, never copied
  __device__ __forceinline__ void at(int panel, TileOperand &op, int &p, int &col) const {
    panel_of(*segs, panel, op, p, col);
  }
  // output column of panel `panel`
  __device__ __forceinline__ int out_col(int panel) const {
    TileOperand op;
    int p, col;
    panel_of(*segs, panel, op, p, col);
    return col + p * 16;
  }
};

// A value known to be wave-uniform, moved to scalar registers.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// A global-memory pointer known to be wave-uniform: scalar registers, and
// the global address space restated so its loads stay global (not flat)
// loads, which would share the wait counter of the LDS lookups.
template <class T>
__device__ __forceinline__ const T *uniform(const T *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  typedef const __attribute__((address_space(1))) T GlobalT;
  return (const T *)(GlobalT *)(((uint64_t)hi << 32) | lo);
}

// The panels of one operand of one expert of a grouped linear (e.g. its
// gate or its up projection, seg_n columns at output column k seg_n): a
// wave's steps never leave its operand, whose addresses are read once into
// scalar registers.
struct ExpertWalk {
  TileOperand op;
  int col;
  __device__ __forceinline__ void load(const ecf8_tile_operand *ops, int k, int seg_n) {
    const ecf8_tile_operand &t = ops[k];
    op = TileOperand{uniform(static_cast<const uint8_t *>(t.stream)), uniform(t.seg_off),
                     uniform(t.gaps), uniform(static_cast<const uint8_t *>(t.other)),
                     uniform(t.weight_scale)};
    col = k * seg_n;
  }
  __device__ __forceinline__ void at(int panel, TileOperand &o, int &p, int &c) const {
    o = op;
    p = panel;
    c = col;
  }
};

// Compiler barrier: memory operations keep their order across it, so loads
// issue in the order their waits are counted in (vmcnt retires in order).
__device__ __forceinline__ void issue_order() { asm volatile("" ::: "memory"); }

// LDS-only workgroup barrier: outstanding global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One step of a hardware wave's walk: a panel of the group's walk and one
// K group of it, kg = v + u * WAVES -- step u of virtual wave v, the wave
// of the FP8 linear that sums group kg (a step past the last group or
// panel computes nothing and reads in-bounds clamped addresses).
// Wave-uniform.
struct Step {
  TileOperand op;
  int p, col;    // panel index inside the operand, its first output column
  int kg;        // group, 0 when past the last one
  int v;         // virtual wave whose partial sums this step adds to
  bool valid;    // a real panel and group: decoded and multiplied
  bool vcloses;  // v's last step of the panel: its partial sums are parked
  bool closes;   // the hardware wave's last step of the panel
};

template <class Walk>
__device__ __forceinline__ Step step_at(const Walk &walk, int panel, int v, int u, int waves,
                                        int kgroups, int n_panels, bool vcloses, bool closes) {
  Step st;
  const int kg = v + u * waves;
  st.valid = panel < n_panels && kg < kgroups;
  st.v = v;
  st.vcloses = vcloses;
  st.closes = closes;
  walk.at(panel < n_panels ? panel : n_panels - 1, st.op, st.p, st.col);
  st.kg = kg < kgroups ? kg : 0;
  return st;
}

// The step's offsets and weight scale by one vector load: lane 0 the
// segment's first byte, lane 1 its end, the other lanes its weight scale.
__device__ __forceinline__ uint32_t step_meta(const Step &st, int kgroups, int lane) {
  const uint32_t s = (uint32_t)st.p * (uint32_t)kgroups + (uint32_t)st.kg;
  const uint32_t *a =
      lane < 2 ? st.op.seg_off + s + lane
               : reinterpret_cast<const uint32_t *>(st.op.ws) + (size_t)(st.p >> 3) * kgroups + st.kg;
  return *a;
}

// Launch shapes: panels of partial sums per reduction (RED) and FP8
// workgroups per workgroup (G), chosen for waves per CU (LDS: automaton
// 24.6 KB + 1 KB staging per wave + RED x waves KB of partial sums; MI355X,
// Qwen3-30B-A3B experts at 16 tokens: down 58.2 us at G = 1, RED = 4 and
// 51.7 us at G = 2, RED = 2).  The sixteen-wave dense shape takes RED = 2:
// 74 KB, two workgroups per CU.
#ifndef ECF8_TILE_DENSE16_RED
#define ECF8_TILE_DENSE16_RED 2
#endif
#ifndef ECF8_TILE_DENSE8_RED
#define ECF8_TILE_DENSE8_RED 2
#endif
#ifndef ECF8_TILE_DENSE8_GROUPS
#define ECF8_TILE_DENSE8_GROUPS 1
#endif
#ifndef ECF8_TILE_MOE8_RED
#define ECF8_TILE_MOE8_RED ECF8_TILE_MOE_RED
#endif
#ifndef ECF8_TILE_MOE_RED
#define ECF8_TILE_MOE_RED 2
#endif
// The eight-wave shapes at G = 1 hold 49.4 KB of LDS: three workgroups per
// CU, six waves per SIMD.  Two FP8 workgroups per workgroup (one automaton
// copy, 74.3 KB) give two workgroups per CU and eight waves per SIMD.  On
// MI355X, alternating builds: Qwen3-30B-A3B grouped gate/up at 16 tokens
// 67.0 / 67.6 us at G = 2 against 69.1 / 71.0 at G = 1 (bit-identical),
// e2e 1651 / 1650 against 1647 / 1646 tokens/s; the dense eight-wave shape
// keeps G = 1: its smallest linear (o, 256 panels) would fill only 128 CUs
// (11.8 -> 14.0 us).
#ifndef ECF8_TILE_MOE8_GROUPS
#define ECF8_TILE_MOE8_GROUPS 2
#endif
#ifndef ECF8_TILE_MOE4_GROUPS
#define ECF8_TILE_MOE4_GROUPS 2
#endif
// Three-wave shape (K = 768: the FP8 grouped linear's three waves of two
// groups each): G = 4, twelve waves -- a multiple of the CU's four SIMDs.
constexpr int kDense16Red = ECF8_TILE_DENSE16_RED;
constexpr int kDense8Red = ECF8_TILE_DENSE8_RED, kMoeRed = ECF8_TILE_MOE_RED;
constexpr int kMoe8Groups = ECF8_TILE_MOE8_GROUPS, kMoe4Groups = ECF8_TILE_MOE4_GROUPS;
constexpr int kDense8Groups = ECF8_TILE_DENSE8_GROUPS, kMoe8Red = ECF8_TILE_MOE8_RED;

// Steps ahead a wave loads a segment's window and nibbles (P) and its
// offsets (at least P + 1).  None and one: the kernel fits 64 VGPRs, so
// the sixteen-wave dense shape runs two workgroups (eight waves per SIMD)
// per CU and the waves hide each other's round trips; the decode is then
// mostly VALU-bound (counters on the Qwen3-8B gate/up at M = 16: VALU busy
// 66 % at four waves per SIMD with a step of prefetch, 74 % at eight
// without).  MI355X, Qwen3-8B layer at M = 16: 77.2 us against 78.5 with a
// step of prefetch (75 VGPRs, four waves per SIMD); offsets two steps ahead
// spill at 64 VGPRs (92.6 us); prefetch distances 2 and 3 at four waves
// per SIMD measured slower still (90.2 and 89.3 us against 81.0 at 1).
#ifndef ECF8_TILE_PREFETCH
#define ECF8_TILE_PREFETCH 0
#endif
constexpr int kPrefetch = ECF8_TILE_PREFETCH;
#ifndef ECF8_TILE_META_AHEAD
#define ECF8_TILE_META_AHEAD 1
#endif
constexpr int kMetaAhead = ECF8_TILE_META_AHEAD;
// Without prefetch, each pass issues the next pass's window right after its
// own decode (it then overlaps the MFMAs and the reduction, and is not live
// across a decode), and the prologue the first one, behind the automaton's
// loads.  MI355X, same-box alternation: Qwen3-8B layer at M = 16 75.1-75.3
// us against 76.1-76.3 with each window issued at its own step; grouped
// down projection 43.4 against 44.3 us (the sixteen-wave shape spills 12
// bytes per lane around the MFMAs and is still faster).
#ifndef ECF8_TILE_LATE
#define ECF8_TILE_LATE 1
#endif
constexpr bool kLateWindow = ECF8_TILE_LATE;
static_assert(kPrefetch >= 0 && kPrefetch <= 3, "prefetch distance");
// Steps a wave decodes at once (interleaved automaton walks), then
// multiplies one after the other in step order.  One: on MI355X two
// measured slower (Qwen3-8B layer at M = 16: 81.9 us at 1, 92.8 at 2;
// Qwen3-30B-A3B down projection 52.3 vs 67.9 us) -- the same VALU work per
// step, 120+ VGPRs (6 -> 4 waves per SIMD where LDS allowed 6) and scalar
// registers spilled to VGPR lanes, for no latency left to hide.
#ifndef ECF8_TILE_PAIR
#define ECF8_TILE_PAIR 1
#endif
constexpr int kPair = ECF8_TILE_PAIR;
static_assert(kPair == 1 || kPair == 2, "steps per pass");
// The sign/mantissa nibbles of a step loaded with its activations, at the
// step itself (1), or a step ahead with its code window (0).
#ifndef ECF8_TILE_OTH_NOW
#define ECF8_TILE_OTH_NOW 0
#endif
constexpr bool kOthNow = ECF8_TILE_OTH_NOW;

// out[m, col + n] = sum_g (sum_{k in g} aq[m,k] * W[n,k]) * as[m,g] * ws[n/128, g]
// for M <= 16, persistent over the 16-column panels.
//
// A workgroup runs G groups of WAVES waves; group g is the FP8
// linear's workgroup number blockIdx.x * G + g of a grid G times larger: it
// takes those panels and sums each in the order of that workgroup's WAVES
// waves, so the result does not depend on G (more waves per CU for shapes
// whose FP8 workgroup is small).  The groups walk in lockstep (a group out
// of panels walks empty steps), so every wave reaches the same barriers.
//
// Hardware wave w of a group is the FP8 linear's wave w (groups w,
// w + WAVES, ...; when WAVES does not divide the groups, the last step of
// some waves is empty).
//
// Each wave walks its steps (segments) as a software pipeline: while it
// decodes step t, the code windows and nibbles of steps t+1..t+P (P =
// kPrefetch) and the offsets of step t+P+1 are in flight -- every load
// unconditional (clamped addresses) and issued in a fixed order, so the wait
// before a decode never covers a later step's loads.  The loop is unrolled
// by P+1 and the buffers rotate by name, so no in-flight register is
// copied.  Partial sums of up to RED panels per group wait in LDS and are
// reduced together, in wave order as the FP8 linear sums them, behind a
// barrier that fences LDS only.  (A barrier-free scheme -- the last wave in
// sums each panel -- measured slower on MI355X: it hands the summing to the
// slowest wave.)
// Arguments of the dense linear (one fused set of operands, rows 0..M-1)
// and of the grouped expert linear (workgroup (split, slot) takes expert
// active[slot], its rows offsets[e].. of the sorted pairs, gathered from
// aq rows row_of[q] when row_of is set).
struct TileDenseArgs {
  const uint8_t *aq;
  const float *as;
  int M, K;
  TileSegs segs;
  const uint32_t *table;
  uint16_t *out;
  int ldo, n_panels;
};

struct TileMoeArgs {
  const uint8_t *aq;
  const float *as;
  const int *row_of;
  const int *offsets;
  const int *active;
  const int *n_active;
  const ecf8_tile_operand *ops;   // [E * n_segs]
  const uint32_t *const *tables;  // [E]
  uint16_t *out;
  int K, ldo, n_segs, seg_n;
  // workgroups per expert: wgs > 0 on a (wgs, experts) grid; wgs = 0 on a
  // one-dimensional grid that the active experts share (gridDim.x /
  // n_active each, a multiple of wgs_unit, at most wgs_cap)
  int wgs, wgs_unit, wgs_cap;
};

// Waves per SIMD the register allocation targets: eight (64 VGPRs), so
// LDS alone bounds the workgroups per CU.
#ifndef ECF8_TILE_WPE
#define ECF8_TILE_WPE 8
#endif
template <int WAVES, int G, int RED, bool kMoe>
__global__ __launch_bounds__(WAVES * G * 64) __attribute__((amdgpu_waves_per_eu(ECF8_TILE_WPE)))
void tile_linear16_kernel(
    typename std::conditional<kMoe, TileMoeArgs, TileDenseArgs>::type a) {
  // P: passes ahead a window is loaded; MD: passes ahead its offsets are
  // (two would keep the offsets a pass reads from being the youngest load,
  // whose wait also waits for the previous pass's output stores, but costs
  // the registers of a second ring entry); NB: buffers of each ring and
  // copies of the unrolled loop
  constexpr int P = kPrefetch, MD = kPrefetch + 1 > kMetaAhead ? kPrefetch + 1 : kMetaAhead;
  constexpr bool kLate = P == 0 && kLateWindow;
  constexpr int HWW = WAVES, NB = kLate ? 2 : MD, HW = HWW * G, S = kPair;
  using Walk = typename std::conditional<kMoe, ExpertWalk, DenseWalk>::type;
  __shared__ uint32_t s_dfa[kDfaEntries + 1];  // + the table's kind word
  __shared__ __attribute__((aligned(16))) uint32_t s_stage[HW][S * kWaveStageDw];
  __shared__ __attribute__((aligned(16))) float s_part[RED][G][WAVES][256];
  const int lane = threadIdx.x & 63;
  const int hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = hw / HWW, hwave = hw % HWW;
  const int K = a.K, kgroups = K / kGroup;
  // The groups of the grid (vgrid of them) are dealt to the operand lanes
  // in equal runs: a grouped linear's operands (e.g. gate, up) one lane
  // each, the host making vgrid a multiple of their count; a dense
  // linear's fused operands one lane.  Group vw takes panels j, j + gpo,
  // ... (j = vw % gpo) of lane vw / gpo, whose tps panels it shares with
  // the lane's other gpo groups.
  int vgrid = (int)gridDim.x * G, vwg0 = (int)blockIdx.x * G;
  int M, row0 = 0, tps, gpo;
  const uint32_t *table;
  Walk walk;
  int slot = 0;
  if constexpr (kMoe) {
    // this workgroup's expert slot and its split of that expert's panels
    const int n_act = uniform(a.n_active[0]);
    int wgs = a.wgs, t = (int)blockIdx.x;
    if (wgs > 0) {
      t += (int)blockIdx.y * wgs;
    } else {
      // as many workgroups per routed expert as the resident grid holds, so
      // that every routed expert's work runs in one round (a fixed split
      // sized for the typical expert count spills a few workgroups into a
      // second round when more experts are routed)
      wgs = n_act > 0 ? (int)gridDim.x / n_act : 1;
      wgs = min(max(wgs / a.wgs_unit, 1) * a.wgs_unit, a.wgs_cap);
    }
    slot = t / wgs;
    vgrid = wgs * G;
    vwg0 = (t - slot * wgs) * G;
  }
  const int vwg = vwg0 + group;
  if constexpr (kMoe) {
    if (slot >= uniform(a.n_active[0])) return;  // uniform, before any barrier
    const int e = uniform(a.active[slot]);
    row0 = uniform(a.offsets[e]);
    // an expert holds at most one pair per routed token: <= 16 rows
    M = min(uniform(a.offsets[e + 1]) - row0, 16);
    table = uniform(a.tables[e]);
    gpo = vgrid / a.n_segs;
    tps = a.seg_n / 16;
    walk.load(a.ops + (size_t)e * a.n_segs, uniform(vwg / gpo), a.seg_n);  // this wave's lane
  } else {
    M = a.M;
    table = a.table;
    walk = DenseWalk{&a.segs};
    gpo = vgrid;
    tps = a.n_panels;
  }
  // group vwg0 + gg's lane and first lane panel, from the workgroup's first
  // group's (one division, in scalars; a dense linear has one lane, gpo =
  // vgrid > every group)
  const int first0 = kMoe ? uniform(vwg0 % gpo) : vwg0, lane0 = kMoe ? uniform(vwg0 / gpo) : 0;
  auto group_start = [&](int gg, int &lane_no) {
    int j = first0 + gg;
    lane_no = lane0;
    if constexpr (kMoe) {
      while (j >= gpo) {  // at most G times
        j -= gpo;
        ++lane_no;
      }
    }
    return j;
  };
  // the workgroup's groups walk in lockstep, as many steps as the one with
  // the most panels
  int most = 0;
#pragma unroll
  for (int gg = 0; gg < G; ++gg) {
    int ln;
    const int j = group_start(gg, ln);
    if (j < tps) most = max(most, (tps - 1 - j) / gpo + 1);
  }
  if (M <= 0 || most == 0) return;  // uniform, before any barrier
  // output column of the o-th panel of group gg, -1 past its last
  auto panel_col = [&](int gg, int o) {
    int ln;
    const int j = group_start(gg, ln) + o * gpo;
    if (j >= tps) return -1;
    if constexpr (kMoe) return ln * a.seg_n + j * 16;
    else return walk.out_col(j);
  };
  uint32_t *const stage = s_stage[hw];
  const float *const as = a.as;

  // the lane's A-operand row and the 4 output rows whose scales it applies;
  // rows past M read the first row: an MFMA output row depends on its own A
  // row only, and rows past M are never stored, so they need no masking
  auto a_row = [&](int rr) -> uint32_t {
    const int q = row0 + (rr < M ? rr : 0);
    if constexpr (kMoe) return (uint32_t)(a.row_of ? a.row_of[q] : q);
    return (uint32_t)q;
  };
  const int r = lane & 15, g = lane >> 4;
  // activations in the tile layout (include/ecf8_llm.h): row R's lane part
  // g of group kg at ((R / 16) * kgroups + kg) * 2048 + (R % 16) * 16 + 256 g
  const uint32_t arow_r = a_row(r);
  const uint32_t aoff = (arow_r >> 4) * (uint32_t)kgroups * 2048u + (arow_r & 15u) * 16u +
                        256u * (uint32_t)g;
  const Rsrc ar = rsrc_at(a.aq), sr = rsrc_at(a.as);
  // byte offsets of the lane's four scale rows
  uint32_t srow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) srow[i] = 4u * a_row(4 * g + i) * (uint32_t)kgroups;
  const int ng = (kgroups + WAVES - 1) / WAVES;
  const int spw = ng;  // steps per panel of each wave
  const int n_real = most * spw;
  // a multiple of NB passes of S steps (trailing ones past the last panel
  // compute nothing), so the unrolled loop's back edge always follows its
  // last copy
  const int n_steps = (n_real + NB * S - 1) / (NB * S) * (NB * S);

  // passes t .. t+MD (S steps each): sc[0..S-1] is the pass being computed
  Step sc[(MD + 1) * S];
  int lane_no;
  int pan = group_start(group, lane_no), q = 0;  // cursor of the step after the last in sc
  auto next_step = [&]() {
    const bool last = q == spw - 1;
    const Step st = step_at(walk, pan, hwave, q, WAVES, kgroups, tps, last, last);
    if (++q == spw) {
      q = 0;
      pan += gpo;
    }
    return st;
  };
#pragma unroll
  for (int i = 0; i < MD * S; ++i) sc[i] = next_step();

  // prologue: offsets of passes 0..MD-1, the automaton table, then the
  // windows and nibbles of passes 0..P-1 -- issued in that order so their
  // round trips overlap
  uint32_t m[NB][S];
  SegLoad w[NB][S];
  u32x4 o[NB][S];
  float wsv[NB][S];
#pragma unroll
  for (int i = 0; i < MD; ++i)
#pragma unroll
    for (int j = 0; j < S; ++j) m[i][j] = step_meta(sc[i * S + j], kgroups, lane);
  issue_order();
  DfaLoad<HW * 64> dfa;
  dfa.load(table, threadIdx.x);
  issue_order();
  auto issue_window = [&](const Step &sl, uint32_t mv, SegLoad &wv, u32x4 &ov, float &sv) {
    const uint32_t si = (uint32_t)sl.p * (uint32_t)kgroups + (uint32_t)sl.kg;
    wv = seg_window(sl.op, si, __builtin_amdgcn_readlane(mv, 0), __builtin_amdgcn_readlane(mv, 1),
                    lane);
    if constexpr (!kOthNow) ov = seg_other(sl.op, si, lane);
    sv = __int_as_float(__builtin_amdgcn_readlane(mv, 2));
  };
#pragma unroll
  for (int i = 0; i < P; ++i)
#pragma unroll
    for (int j = 0; j < S; ++j) issue_window(sc[i * S + j], m[i][j], w[i][j], o[i][j], wsv[i][j]);
  if constexpr (kLate) {
#pragma unroll
    for (int j = 0; j < S; ++j) issue_window(sc[j], m[0][j], w[0][j], o[0][j], wsv[0][j]);
  }
  issue_order();
  dfa.store(s_dfa, threadIdx.x);
  for (int i = lane; i < S * kWaveStageDw; i += 64) stage[i] = 0u;
  lds_barrier();
  if (s_dfa[kDfaEntries] != (uint32_t)ECF8_TABLE_DFA) {
    // not an automaton table (the host cannot see the kind of a table built
    // on the device): every output this group owns becomes a bf16 NaN
    // instead of a product of misread weights.  Uniform, after the last
    // barrier the workgroup passes.
    for (int o = 0;; ++o) {
      const int c = panel_col(group, o);
      if (c < 0) break;
      for (int i = hwave * 64 + lane; i < 16 * M; i += HWW * 64)
        a.out[(size_t)(row0 + (i >> 4)) * a.ldo + c + (i & 15)] = kBf16Nan;
    }
    return;
  }

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  // panels per group waiting in s_part (the same count in every group), and
  // the ordinal of the first
  int pending = 0, first_pending = 0;

  auto reduce = [&]() {
    lds_barrier();
    // item (group gg, panel j, accumulator i) -> one wave (wave-uniform: the
    // panel's operand and columns come from scalar loads); unrolled, as a
    // loop around the store would make the compiler drain the prefetched
    // loads first
    const int per_group = 4 * pending;
#pragma unroll
    for (int k = 0; k < (4 * RED * G + HW - 1) / HW; ++k) {
      const int jw = hw + k * HW;
      if (jw >= G * per_group) break;
      const int gg = jw / per_group, j = (jw % per_group) >> 2, i = jw & 3, l = lane;
      const int c = panel_col(gg, first_pending + j);
      if (c < 0) continue;  // a group out of panels
      float sum = 0.f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) sum += s_part[j][gg][wv][i * 64 + l];
      const int mm = 4 * (l >> 4) + i;
      if (mm < M) a.out[(size_t)(row0 + mm) * a.ldo + c + (l & 15)] = (uint16_t)f32_bf16(sum);
    }
    lds_barrier();
    first_pending += pending;
    pending = 0;
  };

  // pass t (steps t..t+S-1), the k-th copy in the unrolled loop: decode
  // from buffer k, load pass t+P's windows into buffer (k+P) mod NB from
  // their offsets m[(k+P) mod NB], and pass t+P+1's offsets into
  // m[(k+P+1) mod NB]; then the steps' products, in step order
  auto pass = [&](int t, auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr int kl = (k + P) % NB, km = (k + MD) % NB;
    issue_order();
    if constexpr (P == 0 && !kLate) {
      // no prefetch: this pass's windows first, from offsets loaded a pass
      // ago (read into scalars here, before m is reused below)
#pragma unroll
      for (int j = 0; j < S; ++j) issue_window(sc[j], m[k][j], w[k][j], o[k][j], wsv[k][j]);
      issue_order();
    }
    // activations of this pass (L2-resident)
    uint4 av[S][2];
    float sav[S][4];
    u32x4 on[S];
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if constexpr (kOthNow)
        on[j] = seg_other(sc[j].op, (uint32_t)sc[j].p * (uint32_t)kgroups + (uint32_t)sc[j].kg,
                          lane);
      const uint32_t akg = (uint32_t)sc[j].kg * 2048u;
      const u32x4 a0 = __builtin_amdgcn_raw_buffer_load_b128(ar, aoff, akg, 0);
      const u32x4 a1 = __builtin_amdgcn_raw_buffer_load_b128(ar, aoff, akg + 1024u, 0);
      av[j][0] = make_uint4(a0.x, a0.y, a0.z, a0.w);
      av[j][1] = make_uint4(a1.x, a1.y, a1.z, a1.w);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sav[j][i] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(sr, srow[i], 4u * (uint32_t)sc[j].kg, 0));
    }
    issue_order();
#pragma unroll
    for (int j = 0; j < S; ++j) {
      sc[MD * S + j] = next_step();
      m[km][j] = step_meta(sc[MD * S + j], kgroups, lane);
    }
    issue_order();
    if constexpr (P > 0) {
#pragma unroll
      for (int j = 0; j < S; ++j)
        issue_window(sc[P * S + j], m[kl][j], w[kl][j], o[kl][j], wsv[kl][j]);
    }
    issue_order();
    bool any = false;
#pragma unroll
    for (int j = 0; j < S; ++j) any = any || sc[j].valid;
    uint4 ex[S];
    if (any) decode_segments<S>(w[k], s_dfa, stage, lane, ex);
    if constexpr (kLate) {
      // the next pass's windows, into the other buffer: in flight during
      // this pass's MFMAs and reduction
      constexpr int kn = (k + 1) % NB;
      issue_order();
#pragma unroll
      for (int j = 0; j < S; ++j)
        issue_window(sc[MD * S + j], m[kn][j], w[kn][j], o[kn][j], wsv[kn][j]);
      issue_order();
    }
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (sc[j].valid) {
        const uint4 av0 = av[j][0], av1 = av[j][1];
        const u32x4 ok = kOthNow ? on[j] : o[k][j];
        const uint2 w0 = merge8_runs(ex[j].x, ok.x), w1 = merge8_runs(ex[j].y, ok.y);
        const uint2 w2 = merge8_runs(ex[j].z, ok.z), w3 = merge8_runs(ex[j].w, ok.w);
        v4f d = {0.f, 0.f, 0.f, 0.f};
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av0.y << 32) | av0.x), (long)(((uint64_t)w0.y << 32) | w0.x), d, 0,
            0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av0.w << 32) | av0.z), (long)(((uint64_t)w1.y << 32) | w1.x), d, 0,
            0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av1.y << 32) | av1.x), (long)(((uint64_t)w2.y << 32) | w2.x), d, 0,
            0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av1.w << 32) | av1.z), (long)(((uint64_t)w3.y << 32) | w3.x), d, 0,
            0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], sav[j][i] * wsv[k][j], acc[i]);
      }
      if (sc[j].vcloses) {  // the FP8 wave's last step of the panel: park its partial sums
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s_part[pending][group][sc[j].v][i * 64 + lane] = acc[i];
          acc[i] = 0.f;
        }
      }
      if (sc[j].closes) {  // the panel's last step (all groups at once)
        ++pending;
        if (pending == RED || t + j == n_real - 1) reduce();
      }
    }
#pragma unroll
    for (int i = 0; i < MD * S; ++i) sc[i] = sc[i + S];
  };

  for (int t = 0; t < n_steps; t += NB * S) {
    pass(t, std::integral_constant<int, 0>{});
    if constexpr (NB > 1) pass(t + S, std::integral_constant<int, 1 % NB>{});
    if constexpr (NB > 2) pass(t + 2 * S, std::integral_constant<int, 2 % NB>{});
    if constexpr (NB > 3) pass(t + 3 * S, std::integral_constant<int, 3 % NB>{});
  }
}

// Row-major FP8 bytes of tiled operands W[n, K]: every wave decodes
// segments wave_id, + total waves, ... and stores each lane's two 16-byte
// runs.  One operand (kBatch false), or operand blockIdx.y of a device
// array of same-shape operands, each with its own table and output.
struct TileDecodeArgs {
  TileOperand op;
  const uint32_t *table;
  uint8_t *out;
};

struct TileDecodeBatchArgs {
  const ecf8_tile_operand *ops;
  const uint32_t *const *tables;
  uint8_t *const *outs;
};

template <int WAVES, bool kBatch>
__global__ __launch_bounds__(WAVES * 64) void tile_decode_kernel(
    typename std::conditional<kBatch, TileDecodeBatchArgs, TileDecodeArgs>::type a, int K,
    uint32_t n_seg) {
  __shared__ uint32_t s_dfa[kDfaEntries + 1];  // + the table's kind word
  __shared__ __attribute__((aligned(16))) uint32_t s_stage[WAVES][kWaveStageDw];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  TileOperand op;
  const uint32_t *table;
  uint8_t *out;
  if constexpr (kBatch) {
    const ecf8_tile_operand &t = a.ops[blockIdx.y];
    op = TileOperand{static_cast<const uint8_t *>(t.stream), t.seg_off, t.gaps,
                     static_cast<const uint8_t *>(t.other), t.weight_scale};
    table = a.tables[blockIdx.y];
    out = a.outs[blockIdx.y];
  } else {
    op = a.op;
    table = a.table;
    out = a.out;
  }
  load_dfa_batched<WAVES * 64, true>(s_dfa, table, threadIdx.x);
  uint32_t *const stage = s_stage[wave];
  for (int i = lane; i < kWaveStageDw; i += 64) stage[i] = 0u;
  __syncthreads();
  const uint32_t kgroups = (uint32_t)K / kGroup;
  const int r = lane & 15, g = lane >> 4;
  if (s_dfa[kDfaEntries] != (uint32_t)ECF8_TABLE_DFA) {
    // not an automaton table: the segments' bytes become e4m3fn NaNs
    const u32x4 nan4 = {kFp8Nan4, kFp8Nan4, kFp8Nan4, kFp8Nan4};
    for (uint32_t s = blockIdx.x * WAVES + wave; s < n_seg; s += gridDim.x * WAVES) {
      const uint32_t p = s / kgroups, kg = s % kgroups;
      uint8_t *const row = out + (size_t)(p * 16 + r) * K + kg * kGroup + 16 * g;
      *reinterpret_cast<u32x4 *>(row) = nan4;
      *reinterpret_cast<u32x4 *>(row + 64) = nan4;
    }
    return;
  }
  for (uint32_t s = blockIdx.x * WAVES + wave; s < n_seg; s += gridDim.x * WAVES) {
    const SegLoad c = seg_window(op, s, op.seg_off[s], op.seg_off[s + 1], lane);
    const u32x4 oth = seg_other(op, s, lane);
    const uint4 ex = decode_segment(c, s_dfa, stage, lane);
    const uint2 w0 = merge8_runs(ex.x, oth.x), w1 = merge8_runs(ex.y, oth.y);
    const uint2 w2 = merge8_runs(ex.z, oth.z), w3 = merge8_runs(ex.w, oth.w);
    const uint32_t p = s / kgroups, kg = s % kgroups;
    uint8_t *const row = out + (size_t)(p * 16 + r) * K + kg * kGroup + 16 * g;
    __builtin_nontemporal_store(u32x4{w0.x, w0.y, w1.x, w1.y}, reinterpret_cast<u32x4 *>(row));
    __builtin_nontemporal_store(u32x4{w2.x, w2.y, w3.x, w3.y},
                                reinterpret_cast<u32x4 *>(row + 64));
  }
}

inline hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }
inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Workgroups of `kernel` resident on the device at once.
template <class Kernel>
int resident_slots(Kernel kernel, int threads, int64_t *slots) {
  int dev = 0, cus = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void *>(kernel),
                                                    threads, 0) != hipSuccess)
    return ECF8_ERR_HIP;
  *slots = (int64_t)cus * (occ > 0 ? occ : 1);
  return ECF8_OK;
}

template <class Kernel>
int resident_grid(Kernel kernel, int threads, int64_t work, int *grid) {
  int64_t g = 0;
  const int rc = resident_slots(kernel, threads, &g);
  if (rc != ECF8_OK) return rc;
  *grid = (int)(g < work ? g : work);
  return ECF8_OK;
}

int check_operand(const ecf8_tile_operand &t) {
  if (!t.stream || !t.seg_off || !t.gaps || !t.other || !t.weight_scale) return ECF8_ERR_INVALID_ARG;
  if (!aligned(t.stream, 4) || !aligned(t.seg_off, 4) || !aligned(t.gaps, 4) ||
      !aligned(t.other, 16) || !aligned(t.weight_scale, 4))
    return ECF8_ERR_MISALIGNED;
  return ECF8_OK;
}

}  // namespace

extern "C" int ecf8_tile_linear(const void *aq, const float *as, int64_t M, int64_t K,
                                const ecf8_tile_operand *ops, int n_ops, const uint32_t *table,
                                void *out, int64_t ldo, int waves, void *stream) {
  if (!aq || !as || !ops || !table || !out || M <= 0 || K <= 0 || n_ops < 1 ||
      n_ops > ECF8_LINEAR_MAX_SEGS)
    return ECF8_ERR_INVALID_ARG;
  if (M > 16 || K % kGroup || K > (1 << 20) || (waves != 8 && waves != 16))
    return ECF8_ERR_UNSUPPORTED;
  if (!aligned(aq, 16) || !aligned(out, 4) || !aligned(as, 4) || !aligned(table, 4))
    return ECF8_ERR_MISALIGNED;
  TileSegs s{};
  int64_t n_total = 0;
  for (int i = 0; i < n_ops; ++i) {
    const ecf8_tile_operand &t = ops[i];
    const int rc = check_operand(t);
    if (rc != ECF8_OK) return rc;
    if (t.n <= 0 || t.out_col < 0) return ECF8_ERR_INVALID_ARG;
    if (t.n % kGroup) return ECF8_ERR_UNSUPPORTED;
    if (t.out_col + t.n > ldo) return ECF8_ERR_CAPACITY;
    n_total += t.n;
    s.op[i] = TileOperand{static_cast<const uint8_t *>(t.stream), t.seg_off, t.gaps,
                          static_cast<const uint8_t *>(t.other), t.weight_scale};
    s.n_end[i] = (int)n_total;
    s.col[i] = (int)t.out_col;
  }
  if (n_total > (1 << 24)) return ECF8_ERR_UNSUPPORTED;
  s.count = n_ops;
  const int n_panels = (int)(n_total / 16);
  const auto *a = static_cast<const uint8_t *>(aq);
  auto *o = static_cast<uint16_t *>(out);
  const TileDenseArgs args{a, as, (int)M, (int)K, s, table, o, (int)ldo, n_panels};
  int grid = 0, rc;
  if (waves == 16) {
    rc = resident_grid(tile_linear16_kernel<16, 1, kDense16Red, false>, 1024, n_panels, &grid);
    if (rc != ECF8_OK) return rc;
    tile_linear16_kernel<16, 1, kDense16Red, false><<<(unsigned)grid, 1024, 0,
                                                          as_stream(stream)>>>(args);
  } else {
    constexpr int G = kDense8Groups;
    rc = resident_grid(tile_linear16_kernel<8, G, kDense8Red, false>, 512 * G,
                       (n_panels + G - 1) / G, &grid);
    if (rc != ECF8_OK) return rc;
    tile_linear16_kernel<8, G, kDense8Red, false><<<(unsigned)grid, 512 * G, 0,
                                                       as_stream(stream)>>>(args);
  }
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

extern "C" int ecf8_tile_moe_linear(const void *aq, const float *as, const int *row_of,
                                    const int *offsets, const int *active, const int *n_active,
                                    int n_experts, const ecf8_tile_operand *ops,
                                    const uint32_t *const *tables, int n_segs, int64_t seg_n,
                                    int64_t K, int64_t M, void *out, int64_t ldo, int splits,
                                    void *stream) {
  if (!aq || !as || !offsets || !active || !n_active || !ops || !tables || !out ||
      n_experts <= 0 || n_segs < 1 || n_segs > ECF8_LINEAR_MAX_SEGS || seg_n <= 0 || K <= 0 ||
      M <= 0 || splits < 0)
    return ECF8_ERR_INVALID_ARG;
  if (M > 16 || seg_n % kGroup || K % kGroup || K > (1 << 20) || n_segs * seg_n > (1 << 20) ||
      n_experts > 65535)
    return ECF8_ERR_UNSUPPORTED;
  if (ldo < n_segs * seg_n) return ECF8_ERR_CAPACITY;
  if (!aligned(aq, 16) || !aligned(as, 4) || !aligned(out, 4) || !aligned(ops, 8) ||
      !aligned(tables, 8))
    return ECF8_ERR_MISALIGNED;
  const TileMoeArgs args0{static_cast<const uint8_t *>(aq), as, row_of, offsets, active, n_active,
                          ops, tables, static_cast<uint16_t *>(out), (int)K, (int)ldo, n_segs,
                          (int)seg_n, 0, 1, 1};
  const int64_t n_tiles = n_segs * seg_n / 16;
  // the FP8 grouped linear's wave count for this K (it sums in that order)
  const bool eight = K / kGroup > ECF8_MOE_FOUR_WAVE_GROUPS;
  // groups: G FP8 workgroups per workgroup (splits counts FP8 workgroups)
  auto launch = [&](auto kernel, int threads, int groups) {
    TileMoeArgs args = args0;
    // the kernel deals an expert's groups to its operands in equal runs:
    // workgroups per expert a multiple of `unit`
    int unit = 1;
    while ((unit * groups) % n_segs) ++unit;
    const int64_t most = (n_tiles + groups - 1) / groups;  // one panel per group
    args.wgs_unit = unit;
    args.wgs_cap = (int)((most + unit - 1) / unit * unit);
    if (splits > 0) {
      const int64_t g = splits > n_tiles ? n_tiles : splits;
      args.wgs = (int)(((g + groups - 1) / groups + unit - 1) / unit * unit);
      kernel<<<dim3((unsigned)args.wgs, (unsigned)n_experts), threads, 0,
               as_stream(stream)>>>(args);
    } else {
      // one workgroup per resident slot (at least `unit` per expert)
      int64_t slots = 0;
      const int rc = resident_slots(kernel, threads, &slots);
      if (rc != ECF8_OK) return rc;
      const int64_t grid = slots > (int64_t)unit * n_experts ? slots : (int64_t)unit * n_experts;
      args.wgs = 0;
      kernel<<<dim3((unsigned)grid), threads, 0, as_stream(stream)>>>(args);
    }
    return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
  };
  if (eight)
    return launch(tile_linear16_kernel<8, kMoe8Groups, kMoe8Red, true>, 512 * kMoe8Groups,
                  kMoe8Groups);
  // three FP8 waves of two steps (K = 768)
  if (K / kGroup == 6) return launch(tile_linear16_kernel<3, 4, kMoeRed, true>, 768, 4);
  // four FP8 waves of three or four steps (e.g. K = 2048): sixteen waves per
  // workgroup (73 KB of LDS, two per CU).  On MI355X, Qwen3-30B-A3B expert
  // gate/up at 16 tokens: 58.5 us per layer against 58.9 at eight FP8 waves
  if (K / kGroup > 8)
    return launch(tile_linear16_kernel<4, 4, kMoeRed, true>, 1024, 4);
  return launch(tile_linear16_kernel<4, kMoe4Groups, kMoeRed, true>, 256 * kMoe4Groups,
                kMoe4Groups);
}

extern "C" int ecf8_tile_decode(const ecf8_tile_operand *op, int64_t K, const uint32_t *table,
                                void *out, void *stream) {
  if (!op || !table || !out || K <= 0) return ECF8_ERR_INVALID_ARG;
  const int rc0 = check_operand(*op);
  if (rc0 != ECF8_OK) return rc0;
  if (op->n <= 0 || op->n % 16 || K % kGroup) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(out, 16) || !aligned(table, 4)) return ECF8_ERR_MISALIGNED;
  if ((int64_t)op->n * K >= ((int64_t)1 << 40)) return ECF8_ERR_UNSUPPORTED;
  const int64_t n_seg = (int64_t)(op->n / 16) * (K / kGroup);
  if (n_seg > (int64_t)UINT32_MAX / 2) return ECF8_ERR_UNSUPPORTED;
  const TileDecodeArgs args{
      TileOperand{static_cast<const uint8_t *>(op->stream), op->seg_off, op->gaps,
                  static_cast<const uint8_t *>(op->other), op->weight_scale},
      table, static_cast<uint8_t *>(out)};
  int grid = 0;
  const int rc = resident_grid(tile_decode_kernel<8, false>, 512, (n_seg + 7) / 8, &grid);
  if (rc != ECF8_OK) return rc;
  tile_decode_kernel<8, false><<<(unsigned)grid, 512, 0, as_stream(stream)>>>(args, (int)K,
                                                                             (uint32_t)n_seg);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

extern "C" int ecf8_tile_decode_batch(const ecf8_tile_operand *ops, const uint32_t *const *tables,
                                      void *const *outs, int n_ops, int64_t n, int64_t K,
                                      void *stream) {
  if (!ops || !tables || !outs || n_ops <= 0 || n <= 0 || K <= 0) return ECF8_ERR_INVALID_ARG;
  if (n % 16 || K % kGroup || n_ops > 65535) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(ops, 8) || !aligned(tables, 8) || !aligned(outs, 8)) return ECF8_ERR_MISALIGNED;
  if (n * K >= ((int64_t)1 << 40)) return ECF8_ERR_UNSUPPORTED;
  const int64_t n_seg = (n / 16) * (K / kGroup);
  if (n_seg > (int64_t)UINT32_MAX / 2) return ECF8_ERR_UNSUPPORTED;
  const TileDecodeBatchArgs args{ops, tables, reinterpret_cast<uint8_t *const *>(outs)};
  int64_t slots = 0;
  const int rc = resident_slots(tile_decode_kernel<8, true>, 512, &slots);
  if (rc != ECF8_OK) return rc;
  // about two workgroups per resident slot over all operands
  int64_t g = (2 * slots + n_ops - 1) / n_ops, need = (n_seg + 7) / 8;
  g = g < 1 ? 1 : g > need ? need : g;
  tile_decode_kernel<8, true><<<dim3((unsigned)g, (unsigned)n_ops), 512, 0, as_stream(stream)>>>(
      args, (int)K, (uint32_t)n_seg);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}
