// Device helpers shared by the decode kernels (ecf8_decode.hip) and the
// fused decode + linear kernels (ecf8_tile.hip): the byte automaton in LDS,
// the wave64 prefix sum and the exponent / sign-mantissa merge.
#ifndef ECF8_DEV_H
#define ECF8_DEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ecf8_layout.h"

namespace ecf8 {
namespace dev {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// (a & M) | (b & ~M) as one v_bfi_b32.  The constant mask reaches the
// compiler as an opaque SGPR value (one s_mov): with a visible constant it
// expands the expression to ANDs and an OR.  The v_bfi_b32 itself is the
// compiler's own instruction, not inline asm, so the hazard recognizer sees
// its VGPR write -- an MFMA that reads a VGPR right after a VALU op wrote it
// needs wait states the recognizer inserts only for instructions it knows.
template <uint32_t M>
__device__ __forceinline__ uint32_t bfi(uint32_t a, uint32_t b) {
  uint32_t m;
  asm("s_mov_b32 %0, %1" : "=s"(m) : "i"(M));
  return (a & m) | (b & ~m);
}

// 8 FP8 bytes from 8 exponent nibbles (E, element k in bits 4k..4k+3) and
// 4 packed sign/mantissa bytes (O, byte j = o_{2j} << 4 | o_{2j+1}).
__device__ __forceinline__ uint2 merge8(uint32_t e, uint32_t o) {
  // even elements 2j: sign = O_j bit 7, exponent = E_j low nibble,
  // mantissa = O_j bits 4..6
  const uint32_t h = bfi<0x80808080u>(o, bfi<0x78787878u>(e << 3, o >> 4));
  // odd elements 2j+1: sign = O_j bit 3, exponent = E_j high nibble,
  // mantissa = O_j bits 0..2
  const uint32_t l = bfi<0x80808080u>(o << 4, bfi<0x78787878u>(e >> 1, o));
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

// The entry at byte offset `off` of the automaton in LDS.
__device__ __forceinline__ uint32_t dfa_at(const uint32_t *s_dfa, uint32_t off) {
  return *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(s_dfa) + off);
}

// Load a table into the workgroup's LDS automaton.  Fields a well-formed
// table never holds (only a corrupt or mismatched one) are forced into range:
// a row outside the automaton becomes the exact row and a count above 4
// symbols becomes 4, so every lookup stays inside s_dfa and every OR inside
// the staging buffer's spill dwords.
__device__ __forceinline__ uint32_t dfa_entry_in_range(uint32_t e) {
  if ((e & kDfaRowMask) >= ((uint32_t)kDfaRows << 10))
    e = (e & ~kDfaRowMask) | ((uint32_t)kDfaExactRow << 10);
  const uint32_t n4 = min(e & 0xFCu, 4u * kDfaMaxSyms);
  return (e & 0xFFFF7C00u) | n4;
}

// One entry per lane and round trip: for the batched kernel, whose task
// loop keeps more registers live around it.
template <int kThreads>
__device__ __forceinline__ void load_dfa(uint32_t *s_dfa, const uint32_t *__restrict__ table,
                                         int tid) {
  for (int i = tid; i < kDfaEntries; i += kThreads) s_dfa[i] = dfa_entry_in_range(table[i]);
}

// Up to 13 loads per lane in flight before the first wait: at 512 lanes
// the whole table arrives in one memory round trip instead of 13 (measured
// on MI355X: ~3 us less per launch of the one-tensor kernel).
// kWithKind: the table's kind word (index kDfaEntries) is copied unchanged
// into s_dfa[kDfaEntries] (s_dfa then holds kDfaEntries + 1 words).
template <int kThreads, bool kWithKind = false>
__device__ __forceinline__ void load_dfa_batched(uint32_t *s_dfa,
                                                 const uint32_t *__restrict__ table, int tid) {
  constexpr int kWords = kDfaEntries + (kWithKind ? 1 : 0);
  constexpr int kIters = (kWords + kThreads - 1) / kThreads;
  constexpr int kBatch = kIters < 13 ? kIters : 13;
#pragma unroll
  for (int j0 = 0; j0 < kIters; j0 += kBatch) {
    uint32_t v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = tid + (j0 + j) * kThreads;
      v[j] = i < kWords ? table[i] : 0u;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = tid + (j0 + j) * kThreads;
      if (i < kDfaEntries) s_dfa[i] = dfa_entry_in_range(v[j]);
      else if (kWithKind && i == kDfaEntries) s_dfa[i] = v[j];
    }
  }
}

// A pointer read out of memory (a descriptor) to global memory: the
// address space restated, so its loads and stores are global, not flat,
// operations -- flat ones also count on the LDS wait counter, so every LDS
// wait would wait for them too.
template <class T>
__device__ __forceinline__ T *as_global(T *p) {
  typedef __attribute__((address_space(1))) T GlobalT;
  return (T *)(GlobalT *)reinterpret_cast<uint64_t>(p);
}

// load_dfa_batched in rounds of kBatch loads per lane, from a table address
// read out of memory (a descriptor), as buffer loads: one lane offset for
// every round, each round's base in its own buffer resource (scalar, and
// dependent on the table, so a caller's task loop cannot hoist it).  As
// global loads, each round above the first needed its own lane address,
// which the batched kernel's task loop kept live and spilled to scratch,
// reloading them for every task.
template <int kThreads, int kBatch>
__device__ __forceinline__ void load_dfa_rounds(uint32_t *s_dfa, const uint32_t *table, int tid) {
  const uint32_t lane_off = 4u * (uint32_t)tid;
  constexpr int kIters = (kDfaEntries + kThreads - 1) / kThreads;
#pragma unroll
  for (int j0 = 0; j0 < kIters; j0 += kBatch) {
    uint32_t v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = tid + (j0 + j) * kThreads;
      const __amdgpu_buffer_rsrc_t t = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint32_t *>(table + (j0 + j) * kThreads), 0, -1, 0x00020000);
      v[j] = (j0 + j < kIters && i < kDfaEntries)
                 ? __builtin_amdgcn_raw_buffer_load_b32(t, lane_off, 0, 0)
                 : 0u;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = tid + (j0 + j) * kThreads;
      if (j0 + j < kIters && i < kDfaEntries) s_dfa[i] = dfa_entry_in_range(v[j]);
    }
  }
}

// The table in two halves -- loads into registers, then LDS stores -- so a
// kernel can issue other loads in between and overlap their round trips.
template <int kThreads>
struct DfaLoad {
  // the table's kind word (index kDfaEntries) rides with the entries: it
  // lands in s_dfa[kDfaEntries] unchanged, so s_dfa holds kDfaEntries + 1
  static constexpr int kIters = (kDfaEntries + 1 + kThreads - 1) / kThreads;
  uint32_t v[kIters];
  __device__ __forceinline__ void load(const uint32_t *__restrict__ table, int tid) {
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
      const int i = tid + j * kThreads;
      v[j] = i <= kDfaEntries ? table[i] : 0u;
    }
  }
  __device__ __forceinline__ void store(uint32_t *s_dfa, int tid) const {
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
      const int i = tid + j * kThreads;
      if (i < kDfaEntries) s_dfa[i] = dfa_entry_in_range(v[j]);
      else if (i == kDfaEntries) s_dfa[i] = v[j];
    }
  }
};

}  // namespace dev
}  // namespace ecf8

#endif  // ECF8_DEV_H
