// Device construction of a derived decode table: the steps of
// ecf8_table_build.h across one 1024-lane workgroup, so that a table can be
// built on the stream that uses it, without a host round trip (the decode
// launch in the reference's call form, graph capture).  The result is the
// same bytes the host builder writes, kind word included.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ecf8.h"
#include "ecf8_layout.h"
#include "ecf8_table_build.h"

namespace {

using namespace ecf8;

constexpr int kBuildThreads = 1024;
constexpr int kPrefixesPerLane = (kPrefixKeys + kBuildThreads - 1) / kBuildThreads;  // 64
static_assert(kPrefixesPerLane == 64, "one 64-bit mask of prefixes per lane");
static_assert(kTableWords > kKindWord, "the table holds its kind word");

__device__ __forceinline__ int wave_inclusive_sum(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// snap (optional): [n_luts, want_kind, LUT bytes] the table in `table` was
// built from.  When it matches the current LUTs the table is kept as it is;
// otherwise it is rebuilt and snap rewritten (after the comparison, which
// every lane finishes before the barrier that publishes its result).
__global__ __launch_bounds__(kBuildThreads) void build_table_kernel(
    const uint8_t *__restrict__ luts, int n_luts, int want_kind, uint32_t *__restrict__ table,
    uint32_t *__restrict__ snap) {
  __shared__ TableScratch s;
  __shared__ int s_wave_total[kBuildThreads / 64];
  __shared__ int s_fail;
  const int tid = threadIdx.x;
  const uint32_t *l32 = reinterpret_cast<const uint32_t *>(luts);
  uint32_t *s32 = reinterpret_cast<uint32_t *>(s.luts);
  int differs = 0;
  for (int i = tid; i < n_luts * 64; i += kBuildThreads) {
    const uint32_t v = l32[i];
    s32[i] = v;
    if (snap) differs |= snap[2 + i] != v;
  }
  if (tid == 0) {
    s.n_luts = n_luts;
    s_fail = 0;
    if (snap) differs |= snap[0] != (uint32_t)n_luts || snap[1] != (uint32_t)want_kind;
  }
  if (snap) {
    if (!__syncthreads_or(differs)) return;  // uniform: the table is current
    for (int i = tid; i < n_luts * 64; i += kBuildThreads) snap[2 + i] = s32[i];
    if (tid == 0) {
      snap[0] = (uint32_t)n_luts;
      snap[1] = (uint32_t)want_kind;
    }
  }
  __syncthreads();

  bool dfa = want_kind != ECF8_TABLE_MULTI;  // uniform
  if (dfa) {
    // range trees of the second-level rows, then of the first level
    const int rows = second_level_rows(s);
    for (int i = tid; i < rows * 256; i += kBuildThreads)
      s.tree[1 + (i >> 8)][256 + (i & 255)] = tree_leaf(s, 1 + (i >> 8), i & 255);
    __syncthreads();
    for (int half = 128; half >= 1; half >>= 1) {
      for (int i = tid; i < rows * half; i += kBuildThreads) {
        const int t = 1 + i / half, n = half + i % half;
        s.tree[t][n] = tree_combine(s.tree[t][2 * n], s.tree[t][2 * n + 1]);
      }
      __syncthreads();
    }
    if (tid < 256) s.tree[0][256 + tid] = tree_leaf(s, 0, tid);
    __syncthreads();
    for (int half = 128; half >= 1; half >>= 1) {
      if (tid < half) s.tree[0][half + tid] = tree_combine(s.tree[0][2 * (half + tid)],
                                                           s.tree[0][2 * (half + tid) + 1]);
      __syncthreads();
    }
    // pending prefixes in canonical order: lane tid checks indices
    // [64 tid, 64 tid + 64); an exclusive scan of the counts places them
    uint64_t mine = 0;
    for (int j = 0; j < kPrefixesPerLane; ++j) {
      const int idx = tid * kPrefixesPerLane + j;
      if (idx < kPrefixKeys && prefix_pending(s, prefix_key(idx))) mine |= 1ull << j;
    }
    const int cnt = __popcll(mine);
    const int incl = wave_inclusive_sum(cnt);
    if ((tid & 63) == 63) s_wave_total[tid >> 6] = incl;
    __syncthreads();
    int before = incl - cnt, total = 0;
    for (int w = 0; w < kBuildThreads / 64; ++w) {
      const int t = s_wave_total[w];
      if (w < (tid >> 6)) before += t;
      total += t;
    }
    if (total > kDfaMaxPending) {
      dfa = false;  // uniform: every lane read the same totals
    } else {
      while (mine) {
        const int j = __builtin_ctzll(mine);
        mine &= mine - 1;
        s.pending[before++] = prefix_key(tid * kPrefixesPerLane + j);
      }
      if (tid == 0) s.n_pending = total;
    }
    __syncthreads();
    if (dfa) {
      for (int e = tid; e < kDfaEntries; e += kBuildThreads) {
        uint32_t v = 0;
        if (dfa_table_entry(s, e, &v)) table[e] = v;
        else s_fail = 1;
      }
      __syncthreads();
      if (s_fail) dfa = false;
    }
    if (dfa) {
      for (int w = kKindWord + tid; w < kTableWords; w += kBuildThreads)
        table[w] = w == kKindWord ? (uint32_t)ECF8_TABLE_DFA : 0u;
      return;
    }
  }
  if (want_kind == ECF8_TABLE_DFA) {  // the automaton was asked for and is impossible
    if (tid == 0) table[kKindWord] = 0xFFFFFFFFu;
    return;
  }
  for (int w = tid; w < kTableWords; w += kBuildThreads) {
    uint32_t v = 0;
    if (w < kMultiEntries) v = multi_entry(s, w);
    else if (w == kKindWord) v = (uint32_t)ECF8_TABLE_MULTI;
    table[w] = v;
  }
}

}  // namespace

extern "C" int ecf8_build_table(const uint8_t *luts, int n_luts, int want_kind, uint32_t *table,
                                int *table_kind, void *stream) {
  if (!luts || !table) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  if (want_kind != ECF8_TABLE_ANY && want_kind != ECF8_TABLE_MULTI && want_kind != ECF8_TABLE_DFA)
    return ECF8_ERR_INVALID_ARG;
  // a refused automaton is only reported through table_kind
  if (want_kind == ECF8_TABLE_DFA && !table_kind) return ECF8_ERR_INVALID_ARG;
  if (((uintptr_t)luts & 3) || ((uintptr_t)table & 3)) return ECF8_ERR_MISALIGNED;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(build_table_kernel, dim3(1), dim3(kBuildThreads), 0, s, luts, n_luts,
                     want_kind, table, static_cast<uint32_t *>(nullptr));
  if (hipGetLastError() != hipSuccess) return ECF8_ERR_HIP;
  if (!table_kind) return ECF8_OK;
  uint32_t kind = 0;
  if (hipMemcpyAsync(&kind, table + kKindWord, sizeof(kind), hipMemcpyDeviceToHost, s) !=
          hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return ECF8_ERR_HIP;
  if (kind != ECF8_TABLE_DFA && kind != ECF8_TABLE_MULTI) return ECF8_ERR_FORMAT;
  *table_kind = (int)kind;
  return ECF8_OK;
}

extern "C" int ecf8_build_table_cached(const uint8_t *luts, int n_luts, int want_kind, void *cache,
                                       void *stream) {
  if (!luts || !cache) return ECF8_ERR_INVALID_ARG;
  if (n_luts < 2 || n_luts > ECF8_MAX_LUTS) return ECF8_ERR_FORMAT;
  // the kind is only known on the device here, so the automaton cannot be
  // demanded (a refusal could not be reported)
  if (want_kind != ECF8_TABLE_ANY && want_kind != ECF8_TABLE_MULTI) return ECF8_ERR_INVALID_ARG;
  if (((uintptr_t)luts & 3) || ((uintptr_t)cache & 7)) return ECF8_ERR_MISALIGNED;
  static_assert(ECF8_TABLE_BYTES % 8 == 0, "the snapshot follows the table 8-byte aligned");
  auto *table = static_cast<uint32_t *>(cache);
  hipLaunchKernelGGL(build_table_kernel, dim3(1), dim3(kBuildThreads), 0, (hipStream_t)stream,
                     luts, n_luts, want_kind, table, table + ECF8_TABLE_BYTES / 4);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}
