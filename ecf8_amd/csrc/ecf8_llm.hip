// Consumer side of the decode path on gfx950: the block-scaled FP8 linear
// that reads the decoded e4m3fn weights, and the few fused kernels a
// Qwen3-shaped decoder layer needs around it (activation quantization,
// residual + RMSNorm, SiLU gating, per-head norm + rotary embedding + KV
// cache write, split-sequence decode attention).
//
// Numerics follow the fine-grained FP8 scheme of the FP8 checkpoints the
// reference runs (transformers' FP8Linear, used by dfloat/run/run.py's
// DFloatModel for Qwen3-8B-FP8): weights e4m3fn with one fp32 scale per
// 128x128 block, activations quantized on the fly to e4m3fn with one fp32
// scale per row and 128-column group (scale = amax / 448), products
// accumulated in fp32 per 128-column group and scaled by both scales.
//
// Every kernel is deterministic: reductions run in a fixed order, so a
// model decoded from ECF8 and the same model kept in FP8 produce identical
// logits.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ecf8.h"
#include "ecf8_llm.h"

namespace {

constexpr int kGroup = 128;          // quantization group along K
constexpr float kFp8Max = 448.f;     // largest finite e4m3fn value
constexpr int kHeadDim = 128;
constexpr int kAttnChunk = 256;      // positions per attention workgroup

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Tile layout of FP8 operands (activations always, weights optionally; see
// ecf8_llm.h): per 16 rows and 128-column group one 2 KB block in the
// order the MFMA lanes take their operands -- lane l = 16 g + r holds row
// r's bytes [16 g, +16) at byte 16 l and [64 + 16 g, +16) at 1024 + 16 l,
// so each 16-byte load of a wave covers 1 KB contiguous.
// Byte offset of row m's lane-part (g = 0) of group kg:
__device__ __forceinline__ size_t tile_row_off(int m, int kg, int kgroups) {
  return ((size_t)(m >> 4) * kgroups + kg) * 2048 + (size_t)(m & 15) * 16;
}
// ... and of the 16 bytes [16 c, +16) of the group (c = 0..7):
__device__ __forceinline__ size_t tile_chunk_off(int m, int kg, int kgroups, int c) {
  return tile_row_off(m, kg, kgroups) + (size_t)(c >> 2) * 1024 + (size_t)(c & 3) * 256;
}
// Per-lane base of row m's operand bytes (lane part g), to which a group
// adds kg * 2048 and the second half 1024 more.
__device__ __forceinline__ const uint8_t *tile_lane_base(const uint8_t *p, int m, int kgroups,
                                                         int g) {
  return p + tile_row_off(m, 0, kgroups) + (size_t)g * 256;
}

// 16-byte streaming load (weights are read once per launch)
__device__ __forceinline__ uint4 load_stream16(const uint8_t *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16, round to nearest even (the rounding torch uses)
__device__ __forceinline__ uint32_t f32_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// fp32 -> e4m3fn, round to nearest even; |y| is clamped to 448 first, so
// the result is always finite (callers pass values already scaled into
// range).  Subnormals (|y| < 2^-6) have a step of 2^-9.
__device__ __forceinline__ uint32_t f32_e4m3(float y) {
  const uint32_t sign = (__float_as_uint(y) >> 24) & 0x80u;
  const float a = fminf(fabsf(y), kFp8Max);
  uint32_t code;
  if (a < 0.015625f) {
    code = (uint32_t)rintf(a * 512.f);  // 0..8; 8 is the smallest normal
  } else {
    const uint32_t b = __float_as_uint(a);
    const uint32_t e = (b >> 23) - 120u;  // biased e4m3 exponent (bias 7)
    const uint32_t m = b & 0x7fffffu;
    uint32_t q = m >> 20;
    const uint32_t rem = m & 0xfffffu;
    q += (rem > 0x80000u) || (rem == 0x80000u && (q & 1u));
    code = (e << 3) + q;  // a mantissa carry moves into the exponent
  }
  return sign | code;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return __shfl(v, 0);  // every lane takes lane 0's association order
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Quantize 16 consecutive values held by one thread; the 8 threads of a
// 128-column group are 8 consecutive lanes.  Writes 16 e4m3fn bytes and,
// from the group's first thread, the group scale.
__device__ __forceinline__ void quant16(const float (&v)[16], uint8_t *q_out, float *s_out,
                                        bool first_of_group) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  const float s = amax > 0.f ? amax / kFp8Max : 1.f;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w[j] = f32_e4m3(v[4 * j] / s) | (f32_e4m3(v[4 * j + 1] / s) << 8) |
           (f32_e4m3(v[4 * j + 2] / s) << 16) | (f32_e4m3(v[4 * j + 3] / s) << 24);
  }
  *reinterpret_cast<uint4 *>(q_out) = make_uint4(w[0], w[1], w[2], w[3]);
  if (first_of_group) *s_out = s;
}

__device__ __forceinline__ void load16_bf16(const uint16_t *p, float (&v)[16]) {
  const uint4 a = *reinterpret_cast<const uint4 *>(p);
  const uint4 b = *reinterpret_cast<const uint4 *>(p + 8);
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = bf16_f32(w[i] & 0xffffu);
    v[2 * i + 1] = bf16_f32(w[i] >> 16);
  }
}

// ------------------------------------------------------------ FP8 linear

struct LinearSegs {
  const uint8_t *w[ECF8_LINEAR_MAX_SEGS];
  const float *ws[ECF8_LINEAR_MAX_SEGS];
  int n_end[ECF8_LINEAR_MAX_SEGS];  // cumulative output columns
  int col[ECF8_LINEAR_MAX_SEGS];    // first output column of the segment
  int tiled[ECF8_LINEAR_MAX_SEGS];  // weight in the tile layout (else row-major)
  int count;
};

// Buffer resources: a wave-uniform base and extent in scalar registers, so
// a load's address is that base + a scalar offset + one VGPR of 32-bit
// lane offset (a 64-bit address per lane per load would cost the registers
// of a whole batch of loads).  Raw buffer (stride 0); lane offsets at or
// past `bytes` read zero instead of faulting.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
// 16 bytes at lane offset voff + scalar offset soff (kNt: streamed,
// non-temporal -- data read once per launch)
template <bool kNt>
__device__ __forceinline__ uint4 buf_load16(Rsrc r, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNt ? 2 : 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float buf_load_f32(Rsrc r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

// A 16-row panel's weight operand for the lane (r, g), in either weight
// layout: the panel's first byte (wave-uniform: n0 is a multiple of 16),
// the lane's 32-bit offset from it (r K + 16 g row-major, 16 l in the tile
// layout), the step between 128-column groups and the offset of the
// group's second half.  A uniform base and a 32-bit lane offset let each
// load take its address from scalar registers plus one VGPR.
struct WeightLane {
  const uint8_t *base;
  uint32_t lane;
  int step, half;
  __device__ __forceinline__ WeightLane(const uint8_t *w, bool tiled, int n0, int r, int g, int K)
      : base(tiled ? w + (size_t)(n0 >> 4) * (size_t)(K / kGroup) * 2048 : w + (size_t)n0 * K),
        lane(tiled ? 16u * (uint32_t)(16 * g + r) : (uint32_t)r * (uint32_t)K + 16u * (uint32_t)g),
        step(tiled ? 2048 : kGroup),
        half(tiled ? 1024 : 64) {}
  __device__ __forceinline__ const uint8_t *at(int kg) const {
    return base + (size_t)kg * step + lane;
  }
  // the panel as a buffer: 16 rows x K bytes in either layout
  __device__ __forceinline__ Rsrc rsrc(int K) const { return make_rsrc(base, 16u * (uint32_t)K); }
  // group kg's two 16-byte halves (kg wave-uniform), streamed
  __device__ __forceinline__ void load(Rsrc r, int kg, uint4 &lo, uint4 &hi) const {
    lo = buf_load16<true>(r, lane, (uint32_t)kg * (uint32_t)step);
    hi = buf_load16<true>(r, lane, (uint32_t)kg * (uint32_t)step + (uint32_t)half);
  }
};

// out[m, col + n] = sum_g (sum_{k in g} aq[m,k] * w[n,k]) * as[m,g] * ws[n/128, g]
//
// ------------------------------------------------ prompt-size GEMM (M > 16)
//
// out[m, col + n] = sum_g (sum_{k in g} aq[m,k] * w[n,k]) * as[m,g] * ws[n/128, g]
// for M > 16: 128 x 128 output tiles per 256-lane workgroup (2 x 2 waves of
// 64 x 64), one 128-column K group per step through a two-stage LDS ring.
//
// Every operand block -- 16 rows x one K group, 2 KB -- lands in LDS in
// the tile layout of ecf8_llm.h straight from global memory
// (global_load_lds_dwordx4: each lane's 16 bytes to LDS at 16 x lane, no
// register staging): the tile-layout activations and weights block by
// block, row-major weights gathered into the same order.  The MFMA is
// gfx950's v_mfma_f32_16x16x128_f8f6f4 (one instruction per 16 x 16 tile
// and K group): lane l = 16 g + r feeds it the 32 bytes of row r at block
// bytes 16 l and 1024 + 16 l of both operands -- the same K positions for
// both, so the dot product is that of the group -- and each LDS read is 16
// consecutive bytes per lane (conflict-free).  Each group's product is
// scaled by as[m, g] * ws[n/128, g] and added to the fp32 accumulators in
// group order.  Rows past M read the last valid 16-row block and are never
// stored.  Workgroups are ordered so each XCD (blockIdx.x mod 8) takes a
// contiguous run of tiles, column block by column block: the weight block
// a tile column reads stays in that XCD's L2 across its row blocks.
typedef int v8i __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void lds_load16(const uint8_t *g, void *lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void *g, void *lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 4, 0, 0);
}
// Workgroup barrier without a memory fence (a fence on LDS would also wait
// for every stage's loads in flight: they write LDS and are counted by
// vmcnt).  Each wave waits for its own loads of the stage it is about to
// read with an explicit vmcnt first; the empty asm keeps the compiler from
// moving memory operations across the barrier.
__device__ __forceinline__ void gemm_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 bytes of LDS at byte offset `off` + the immediate O of a stage, read
// by inline asm: the compiler cannot see that it reads LDS, so it does not
// wait for the loads still filling the other stages (the caller waits for
// lgkmcnt before using the result).
template <int O>
__device__ __forceinline__ uint4 lds_read16(uint32_t off) {
  uint4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(off), "i"(O));
  return r;
}

#ifndef ECF8_GEMM_BM
#define ECF8_GEMM_BM 256
#endif
constexpr int kGemmBM = ECF8_GEMM_BM;        // tile rows: 2 x 64 per wave row pair
constexpr int kGemmBN = 128;                 // tile columns
constexpr int kGemmWaves = kGemmBM / 32;     // (BM / 64) x 2 waves of 64 x 64
constexpr int kGemmABlocks = kGemmBM / 16, kGemmBBlocks = kGemmBN / 16;
constexpr int kGemmStages = 3;
// loads per wave and stage: A and B block halves, and one of scales
constexpr int kGemmLoads = 2 * (kGemmABlocks + kGemmBBlocks) / kGemmWaves + 1;
// one stage: A blocks, B blocks, A scales
constexpr int kGemmStageBytes = (kGemmABlocks + kGemmBBlocks) * 2048 + kGemmBM * 4;
static_assert(kGemmABlocks % kGemmWaves == 0 && kGemmBBlocks % kGemmWaves == 0,
              "blocks deal evenly to the waves");
static_assert(kGemmLoads < 64, "vmcnt immediate");

__global__ __launch_bounds__(kGemmWaves * 64) void fp8_gemm_kernel(
    const uint8_t *__restrict__ aq, const float *__restrict__ as, int M, int K, LinearSegs segs,
    uint16_t *__restrict__ out, int ldo, int n_mb, int n_tiles) {
  __shared__ __attribute__((aligned(16))) uint8_t s_ring[kGemmStages * kGemmStageBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int kgroups = K / kGroup;

  // tile order: XCD x = blockIdx.x % 8 takes tiles [x * per, (x + 1) * per)
  int tile = blockIdx.x;
  const int per = n_tiles / 8;
  if (tile < 8 * per) tile = (tile % 8) * per + tile / 8;
  const int mb = tile % n_mb, nb = tile / n_mb;
  const int m0 = mb * kGemmBM;

  int n0 = nb * kGemmBN;
  const uint8_t *w = segs.w[0];
  const float *ws = segs.ws[0];
  int col = segs.col[0], seg_start = 0, wt = segs.tiled[0];
#pragma unroll
  for (int s = 1; s < ECF8_LINEAR_MAX_SEGS; ++s) {
    if (s < segs.count && n0 >= segs.n_end[s - 1]) {
      w = segs.w[s];
      ws = segs.ws[s];
      col = segs.col[s];
      wt = segs.tiled[s];
      seg_start = segs.n_end[s - 1];
    }
  }
  n0 -= seg_start;
  typedef const __attribute__((address_space(4))) float ConstF;  // scalar loads
  ConstF *const wsrow = (ConstF *)(ws + (size_t)(n0 / kGroup) * kgroups);
  const int last_rb = (M + 15) / 16 - 1;  // the last 16-row block of aq
  const uint32_t ring = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)s_ring;

  // loads of group kg into stage st: wave v fills A blocks v A/W.. and B
  // blocks v B/W.. (A/W, B/W blocks per wave) and the scales of rows 32 v ..
  // 32 v + 31 (lanes 0..31)
  auto issue = [&](int st, int kg) {
    uint8_t *const sa = s_ring + st * kGemmStageBytes;
    uint8_t *const sb = sa + kGemmABlocks * 2048;
    float *const ss = reinterpret_cast<float *>(sb + kGemmBBlocks * 2048);
    constexpr int na = kGemmABlocks / kGemmWaves, nbk = kGemmBBlocks / kGemmWaves;
#pragma unroll
    for (int h = 0; h < na; ++h) {
      const int t = na * wave + h;
      const int rb = min(m0 / 16 + t, last_rb);
      const uint8_t *ab = aq + ((size_t)rb * kgroups + kg) * 2048;
      lds_load16(ab + 16 * lane, sa + t * 2048);
      lds_load16(ab + 1024 + 16 * lane, sa + t * 2048 + 1024);
    }
#pragma unroll
    for (int h = 0; h < nbk; ++h) {
      const int t = nbk * wave + h;
      const uint8_t *b0, *b1;
      if (wt) {
        const uint8_t *bb = w + ((size_t)(n0 / 16 + t) * kgroups + kg) * 2048;
        b0 = bb + 16 * lane;
        b1 = bb + 1024 + 16 * lane;
      } else {
        b0 = w + (size_t)(n0 + 16 * t + (lane & 15)) * K + kg * kGroup + 16 * (lane >> 4);
        b1 = b0 + 64;
      }
      lds_load16(b0, sb + t * 2048);
      lds_load16(b1, sb + t * 2048 + 1024);
    }
    if (lane < 32) {
      const int row = min(m0 + 32 * wave + lane, M - 1);
      lds_load4(as + (size_t)row * kgroups + kg, ss + 32 * wave);
    }
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // the lane's LDS offsets in a stage: its A, B and scale reads
  const uint32_t a_off = (uint32_t)(4 * wm) * 2048u + 16u * (uint32_t)lane;
  const uint32_t b_off = (uint32_t)(kGemmABlocks + 4 * wn) * 2048u + 16u * (uint32_t)lane;
  const uint32_t s_off =
      (uint32_t)(kGemmABlocks + kGemmBBlocks) * 2048u + 4u * (64u * wm + 4u * (lane >> 4));

  issue(0, 0);
  if (kgroups > 1) issue(1, 1);
  for (int kg = 0; kg < kgroups; ++kg) {
    const int st = kg % kGemmStages;
    // this stage's loads are done unless it is the last: the next one's
    // kGemmLoads may stay in flight
    if (kg + 1 < kgroups)
      __builtin_amdgcn_s_waitcnt((kGemmLoads & 15) | ((kGemmLoads >> 4) << 14) | (0x7 << 4) |
                                 (0xF << 8));
    else
      __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));  // vmcnt(0)
    // every wave's loads of stage st are in LDS, and every wave is done
    // reading the stage refilled below (read in the previous step)
    gemm_barrier();
    const uint32_t base = ring + (uint32_t)st * kGemmStageBytes;
    uint4 al[4], ah[4], bl[4], bh[4], sv[4];
    al[0] = lds_read16<0>(base + a_off);
    ah[0] = lds_read16<1024>(base + a_off);
    al[1] = lds_read16<2048>(base + a_off);
    ah[1] = lds_read16<3072>(base + a_off);
    al[2] = lds_read16<4096>(base + a_off);
    ah[2] = lds_read16<5120>(base + a_off);
    al[3] = lds_read16<6144>(base + a_off);
    ah[3] = lds_read16<7168>(base + a_off);
    bl[0] = lds_read16<0>(base + b_off);
    bh[0] = lds_read16<1024>(base + b_off);
    bl[1] = lds_read16<2048>(base + b_off);
    bh[1] = lds_read16<3072>(base + b_off);
    bl[2] = lds_read16<4096>(base + b_off);
    bh[2] = lds_read16<5120>(base + b_off);
    bl[3] = lds_read16<6144>(base + b_off);
    bh[3] = lds_read16<7168>(base + b_off);
    sv[0] = lds_read16<0>(base + s_off);
    sv[1] = lds_read16<64>(base + s_off);
    sv[2] = lds_read16<128>(base + s_off);
    sv[3] = lds_read16<192>(base + s_off);
    const float sw = wsrow[kg];
    __builtin_amdgcn_s_waitcnt((0x3F & 15) | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));  // lgkmcnt(0)
    // the stage read in the previous step is free: group kg + 2 goes there
    if (kg + 2 < kgroups) issue((kg + 2) % kGemmStages, kg + 2);
    v8i a[4], b[4];
    v4f c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = v8i{(int)al[i].x, (int)al[i].y, (int)al[i].z, (int)al[i].w,
                 (int)ah[i].x, (int)ah[i].y, (int)ah[i].z, (int)ah[i].w};
      b[i] = v8i{(int)bl[i].x, (int)bl[i].y, (int)bl[i].z, (int)bl[i].w,
                 (int)bh[i].x, (int)bh[i].y, (int)bh[i].z, (int)bh[i].w};
      c[i] = v4f{__uint_as_float(sv[i].x) * sw, __uint_as_float(sv[i].y) * sw,
                 __uint_as_float(sv[i].z) * sw, __uint_as_float(sv[i].w) * sw};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f z = {0.f, 0.f, 0.f, 0.f};
        // scale operands 0: the unscaled e4m3 x e4m3 form
        const v4f d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i], b[j], z, 0, 0, 0, 0,
                                                                        0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[i][j][q] = fmaf(d[q], c[i][q], acc[i][j][q]);
      }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = m0 + 64 * wm + 16 * i + 4 * (lane >> 4) + q;
      if (m < M) {
        uint16_t *o = out + (size_t)m * ldo + col + n0 + 64 * wn + (lane & 15);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[16 * j] = (uint16_t)f32_bf16(acc[i][j][q]);
      }
    }
}

// Small-M form (M <= 16, the decode step): one 16-row MFMA tile per
// workgroup of WAVES waves, wave w taking the K groups w, w + WAVES, ... in
// batches of 4 and summing each group with four v_mfma_f32_16x16x32_fp8_fp8:
// lane l = 16 g + r holds row r of both operands, bytes [16 g, +16) and
// [64 + 16 g, +16) of the group -- the 16-byte halves at block bytes 16 l
// and 1024 + 16 l of the tile layout -- so each 16-byte load feeds two
// MFMAs; the K order inside a group is a permutation shared by both
// operands, so the dot product is unchanged.  Every load a batch needs
// (weights from HBM, activations and both scales from L2) is issued before
// its first MFMA, so a batch costs one memory round trip; the loads are
// buffer loads from scalar bases (96 VGPRs for a batch, no spills).  The
// waves' sums meet in LDS and are added in wave order.
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void fp8_linear16_kernel(
    const uint8_t *__restrict__ aq, const float *__restrict__ as, int M, int K, LinearSegs segs,
    uint16_t *__restrict__ out, int ldo) {
  static_assert(WAVES >= 4, "the final sums take one thread each of the first 256");
  __shared__ float red[WAVES][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kgroups = K / kGroup;

  int n0 = blockIdx.x * 16;
  const uint8_t *w = segs.w[0];
  const float *ws = segs.ws[0];
  int col = segs.col[0], seg_start = 0, wt = segs.tiled[0];
#pragma unroll
  for (int s = 1; s < ECF8_LINEAR_MAX_SEGS; ++s) {
    if (s < segs.count && n0 >= segs.n_end[s - 1]) {
      w = segs.w[s];
      ws = segs.ws[s];
      col = segs.col[s];
      wt = segs.tiled[s];
      seg_start = segs.n_end[s - 1];
    }
  }
  n0 -= seg_start;

  const int r = lane & 15, g = lane >> 4;
  const WeightLane wl(w, wt != 0, n0, r, g, K);
  const float *wsrow = ws + (size_t)(n0 / kGroup) * kgroups;
  // An MFMA output row depends on its own A row and scale only, and rows
  // past M are never stored: the pad rows of the tile-layout activations
  // are multiplied as they are, and output rows past M take row M-1's
  // scale (an in-bounds read).
  // buffers: the panel's weights, the first 16-row tile of the
  // activations, their scales (M rows); lane offsets: the lane's activation
  // bytes in a group block, the scale rows it applies
  const Rsrc wr = wl.rsrc(K);
  const Rsrc ar = make_rsrc(aq, (uint32_t)kgroups * 2048u);
  const Rsrc sr = make_rsrc(as, 4u * (uint32_t)M * (uint32_t)kgroups);
  const uint32_t alane = 16u * (uint32_t)lane;
  uint32_t srow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) srow[i] = 4u * (uint32_t)min(4 * g + i, M - 1) * (uint32_t)kgroups;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  constexpr int kU = 4;
  for (int kb = wave; kb < kgroups; kb += WAVES * kU) {
    uint4 wv[kU][2], av[kU][2];
    float wsv[kU], sav[kU][4];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kg = kb + WAVES * u;
      if (kg < kgroups) {
        wl.load(wr, kg, wv[u][0], wv[u][1]);
        wsv[u] = wsrow[kg];
        av[u][0] = buf_load16<false>(ar, alane, (uint32_t)kg * 2048u);
        av[u][1] = buf_load16<false>(ar, alane, (uint32_t)kg * 2048u + 1024u);
#pragma unroll
        for (int i = 0; i < 4; ++i) sav[u][i] = buf_load_f32(sr, srow[i], 4u * (uint32_t)kg);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kg = kb + WAVES * u;
      if (kg >= kgroups) break;
      v4f d = {0.f, 0.f, 0.f, 0.f};
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][0].y << 32) | av[u][0].x),
          (long)(((uint64_t)wv[u][0].y << 32) | wv[u][0].x), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][0].w << 32) | av[u][0].z),
          (long)(((uint64_t)wv[u][0].w << 32) | wv[u][0].z), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][1].y << 32) | av[u][1].x),
          (long)(((uint64_t)wv[u][1].y << 32) | wv[u][1].x), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][1].w << 32) | av[u][1].z),
          (long)(((uint64_t)wv[u][1].w << 32) | wv[u][1].z), d, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], sav[u][i] * wsv[u], acc[i]);
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int i = threadIdx.x >> 6, l = threadIdx.x & 63;
    float sum = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) sum += red[wv][i][l];
    const int m = 4 * (l >> 4) + i;
    if (m < M) out[(size_t)m * ldo + col + n0 + (l & 15)] = (uint16_t)f32_bf16(sum);
  }
}

// Persistent small-M form for K = 4096 (32 groups, 4 per wave): each
// workgroup keeps its waves' activation groups and scales in registers and
// walks the 16-column tiles blockIdx.x, + gridDim.x, ...; the next tile's
// weights are loaded while the current tile's MFMAs run.  Used when there
// are more tiles than resident workgroups (the gate/up projection).
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void fp8_linear16p_kernel(
    const uint8_t *__restrict__ aq, const float *__restrict__ as, int M, LinearSegs segs,
    uint16_t *__restrict__ out, int ldo, int n_tiles) {
  constexpr int K = 4096, kgroups = K / kGroup, kU = kgroups / WAVES;
  static_assert(WAVES >= 4, "the final sums take one thread each of the first 256");
  __shared__ float red[WAVES][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const bool row_ok = r < M;

  // this wave's groups: wave, wave + WAVES, ...
  uint4 av[kU][2];
  float sav[kU][4];
  {
    const uint8_t *arow = tile_lane_base(aq, r, kgroups, g);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kg = wave + WAVES * u;
      av[u][0] = *reinterpret_cast<const uint4 *>(arow + (size_t)kg * 2048);
      av[u][1] = *reinterpret_cast<const uint4 *>(arow + (size_t)kg * 2048 + 1024);
      if (!row_ok) av[u][0] = av[u][1] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mi = 4 * g + i;
        const float v = as[(size_t)(mi < M ? mi : 0) * kgroups + kg];
        sav[u][i] = mi < M ? v : 0.f;
      }
    }
  }

  auto tile_base = [&](int tile, const uint8_t *&w, const float *&ws, int &col, int &n0,
                       int &wt) {
    n0 = tile * 16;
    w = segs.w[0];
    ws = segs.ws[0];
    col = segs.col[0];
    wt = segs.tiled[0];
    int seg_start = 0;
#pragma unroll
    for (int s2 = 1; s2 < ECF8_LINEAR_MAX_SEGS; ++s2) {
      if (s2 < segs.count && n0 >= segs.n_end[s2 - 1]) {
        w = segs.w[s2];
        ws = segs.ws[s2];
        col = segs.col[s2];
        wt = segs.tiled[s2];
        seg_start = segs.n_end[s2 - 1];
      }
    }
    n0 -= seg_start;
  };
  auto load_w = [&](int tile, uint4 (&wv)[kU][2], float (&wsv)[kU]) {
    const uint8_t *w;
    const float *ws;
    int col, n0, wt;
    tile_base(tile, w, ws, col, n0, wt);
    const WeightLane wl(w, wt != 0, n0, r, g, K);
    const Rsrc wr = wl.rsrc(K);
    const float *wsrow = ws + (size_t)(n0 / kGroup) * kgroups;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kg = wave + WAVES * u;
      wl.load(wr, kg, wv[u][0], wv[u][1]);
      wsv[u] = wsrow[kg];
    }
  };

  uint4 wcur[kU][2], wnxt[kU][2];
  float scur[kU], snxt[kU];
  int tile = blockIdx.x;
  if (tile >= n_tiles) return;  // uniform
  load_w(tile, wcur, scur);
  for (;;) {
    const int next = tile + (int)gridDim.x;
    const bool more = next < n_tiles;  // uniform
    if (more) load_w(next, wnxt, snxt);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      v4f d = {0.f, 0.f, 0.f, 0.f};
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][0].y << 32) | av[u][0].x),
          (long)(((uint64_t)wcur[u][0].y << 32) | wcur[u][0].x), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][0].w << 32) | av[u][0].z),
          (long)(((uint64_t)wcur[u][0].w << 32) | wcur[u][0].z), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][1].y << 32) | av[u][1].x),
          (long)(((uint64_t)wcur[u][1].y << 32) | wcur[u][1].x), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
          (long)(((uint64_t)av[u][1].w << 32) | av[u][1].z),
          (long)(((uint64_t)wcur[u][1].w << 32) | wcur[u][1].z), d, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], sav[u][i] * scur[u], acc[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    if (threadIdx.x < 256) {
      const int i = threadIdx.x >> 6, l = threadIdx.x & 63;
      float sum = 0.f;
#pragma unroll
      for (int wv2 = 0; wv2 < WAVES; ++wv2) sum += red[wv2][i][l];
      const int m = 4 * (l >> 4) + i;
      const uint8_t *w;
      const float *ws;
      int col, n0, wt;
      tile_base(tile, w, ws, col, n0, wt);
      if (m < M) out[(size_t)m * ldo + col + n0 + (l & 15)] = (uint16_t)f32_bf16(sum);
    }
    if (!more) break;
    __syncthreads();  // red is rewritten by the next tile
    tile = next;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      wcur[u][0] = wnxt[u][0];
      wcur[u][1] = wnxt[u][1];
      scur[u] = snxt[u];
    }
  }
}

// ------------------------------------------------- quantizing row kernels

// residual += x (if x); y = residual * rsqrt(mean(residual^2) + eps) * w;
// y -> bf16 (ob), and/or -> e4m3fn + group scales (oq, os; from the
// bf16-rounded y when both are written).  One workgroup per row of
// K = 16 * kThreads (4096: 256 threads, 2048: 128), 16 values per thread.
template <int kThreads>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                           float *__restrict__ res,
                                                           const uint16_t *__restrict__ w,
                                                           float eps, int K,
                                                           uint8_t *__restrict__ oq,
                                                           float *__restrict__ os,
                                                           uint16_t *__restrict__ ob) {
  static_assert(kThreads == 128 || kThreads == 256, "rows of 2048 or 4096");
  __shared__ float part[kThreads / 64];
  const int m = blockIdx.x, t = threadIdx.x;
  const size_t base = (size_t)m * K + 16 * t;
  float v[16];
  float4 *rp = reinterpret_cast<float4 *>(res + base);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float4 f = rp[j];
    v[4 * j] = f.x;
    v[4 * j + 1] = f.y;
    v[4 * j + 2] = f.z;
    v[4 * j + 3] = f.w;
  }
  if (x) {
    float xv[16];
    load16_bf16(x + base, xv);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] += xv[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) rp[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ss = fmaf(v[i], v[i], ss);
  ss = wave_sum(ss);
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  float total;
  if constexpr (kThreads == 256)
    total = (part[0] + part[1]) + (part[2] + part[3]);
  else
    total = part[0] + part[1];
  const float rs = rsqrtf(total / (float)K + eps);
  float wv[16];
  load16_bf16(w + 16 * t, wv);
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = v[i] * rs * wv[i];
  if (ob) {
    uint32_t p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = f32_bf16(v[2 * i]) | (f32_bf16(v[2 * i + 1]) << 16);
    uint4 *op = reinterpret_cast<uint4 *>(ob + base);
    op[0] = make_uint4(p[0], p[1], p[2], p[3]);
    op[1] = make_uint4(p[4], p[5], p[6], p[7]);
    if (oq) {  // both outputs: quantize the bf16-rounded values
      float r[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        r[2 * i] = bf16_f32(p[i] & 0xffffu);
        r[2 * i + 1] = bf16_f32(p[i] >> 16);
      }
      quant16(r, oq + tile_chunk_off(m, t >> 3, K / kGroup, t & 7),
              os + (size_t)m * (K / kGroup) + (t >> 3), (t & 7) == 0);
    }
  } else {
    quant16(v, oq + tile_chunk_off(m, t >> 3, K / kGroup, t & 7),
            os + (size_t)m * (K / kGroup) + (t >> 3), (t & 7) == 0);
  }
}

// h = silu(gate) * up over [M, 2I] (gate columns [0, I), up [I, 2I)),
// quantized; grid (ceil(I / 4096), M).  I is a multiple of 128, so the 8
// threads of a group are all inside the row or all past it.
__global__ __launch_bounds__(256) void silu_mul_quant_kernel(const uint16_t *__restrict__ gu, int I,
                                                             uint8_t *__restrict__ oq,
                                                             float *__restrict__ os) {
  const int m = blockIdx.y, e = blockIdx.x * 4096 + 16 * threadIdx.x;
  if (e >= I) return;
  float g[16], u[16];
  load16_bf16(gu + (size_t)m * 2 * I + e, g);
  load16_bf16(gu + (size_t)m * 2 * I + I + e, u);
#pragma unroll
  for (int i = 0; i < 16; ++i) g[i] = g[i] / (1.f + expf(-g[i])) * u[i];
  quant16(g, oq + tile_chunk_off(m, e >> 7, I / kGroup, (e >> 4) & 7),
          os + (size_t)m * (I / kGroup) + (e >> 7), (threadIdx.x & 7) == 0);
}

// plain bf16 -> e4m3fn per 1x128 group; grid (ceil(K / 4096), M), K a
// multiple of 128
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t *__restrict__ x, int K,
                                                        uint8_t *__restrict__ oq,
                                                        float *__restrict__ os) {
  const int m = blockIdx.y, e = blockIdx.x * 4096 + 16 * threadIdx.x;
  if (e >= K) return;
  float v[16];
  load16_bf16(x + (size_t)m * K + e, v);
  quant16(v, oq + tile_chunk_off(m, e >> 7, K / kGroup, (e >> 4) & 7),
          os + (size_t)m * (K / kGroup) + (e >> 7), (threadIdx.x & 7) == 0);
}

// --------------------------------------------- per-head norm + rotary + KV

// One wave, one head row of 128 bf16 values (lane l holds dims 2l, 2l+1):
// RMSNorm over the head (bf16 weights nw), then the rotary embedding at
// position p (rotate-half convention, cos/sin tables [Lmax, 64]); returns
// the lane's two results as packed bf16.
__device__ __forceinline__ uint32_t norm_rope_pair(uint32_t x2, const uint16_t *__restrict__ nw,
                                                   float eps, const float *__restrict__ cosv,
                                                   const float *__restrict__ sinv, int p,
                                                   int lane) {
  float x0 = bf16_f32(x2 & 0xffffu), x1 = bf16_f32(x2 >> 16);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rs = rsqrtf(ss / (float)kHeadDim + eps);
  const uint32_t w2 = *reinterpret_cast<const uint32_t *>(nw + 2 * lane);
  x0 = x0 * rs * bf16_f32(w2 & 0xffffu);
  x1 = x1 * rs * bf16_f32(w2 >> 16);
  const float y0 = __shfl_xor(x0, 32), y1 = __shfl_xor(x1, 32);  // dims d +- 64
  const int j = (2 * lane) & 63;
  const float c0 = cosv[p * 64 + j], c1 = cosv[p * 64 + j + 1];
  const float s0 = sinv[p * 64 + j], s1 = sinv[p * 64 + j + 1];
  const float sg = lane < 32 ? -1.f : 1.f;
  x0 = x0 * c0 + sg * y0 * s0;
  x1 = x1 * c1 + sg * y1 * s1;
  return f32_bf16(x0) | (f32_bf16(x1) << 16);
}

// One wave per (token, head) of the fused qkv projection output
// [B*T, (Hq + 2 Hkv) * 128]: q and k heads get RMSNorm over the head
// (weights qn / kn) and the rotary embedding at position pos[0] + t
// (rotate-half convention, cos/sin tables [Lmax, 64]); q goes to
// q_out [B, Hq, T, 128], k and v to the caches [B, Hkv, Lmax, 128].
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t *__restrict__ qkv, int T, int Hq, int Hkv, const uint16_t *__restrict__ qn,
    const uint16_t *__restrict__ kn, float eps, const float *__restrict__ cosv,
    const float *__restrict__ sinv, const int *__restrict__ pos, int Lmax,
    uint16_t *__restrict__ q_out, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    int n_items) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= n_items) return;
  const int H = Hq + 2 * Hkv;
  const int tok = item / H, hh = item % H;
  const int b = tok / T, t = tok % T;
  const int p = pos[0] + t;
  if (p < 0 || p >= Lmax) return;
  const uint32_t x2 = *reinterpret_cast<const uint32_t *>(qkv + (size_t)tok * H * kHeadDim +
                                                          hh * kHeadDim + 2 * lane);
  const uint32_t outw =
      hh >= Hq + Hkv ? x2 : norm_rope_pair(x2, hh < Hq ? qn : kn, eps, cosv, sinv, p, lane);
  uint16_t *dst;
  if (hh < Hq) {
    dst = q_out + (((size_t)b * Hq + hh) * T + t) * kHeadDim;
  } else if (hh < Hq + Hkv) {
    dst = kc + (((size_t)b * Hkv + (hh - Hq)) * Lmax + p) * kHeadDim;
  } else {
    dst = vc + (((size_t)b * Hkv + (hh - Hq - Hkv)) * Lmax + p) * kHeadDim;
  }
  *reinterpret_cast<uint32_t *>(dst + 2 * lane) = outw;
}

// ------------------------------------------------------ decode attention

// Merge the splits [0, used) of one (b, head) (partials m, l [B*Hq, S] and
// acc [B*Hq, S, 128]) and write the head's 128 outputs: quantized as one
// o-projection group, and optionally as bf16.  One wave, two dims per lane.
__device__ __forceinline__ void combine_head(const float *__restrict__ wm,
                                             const float *__restrict__ wl,
                                             const float *__restrict__ wacc, size_t bh, int S,
                                             int used, int lane, int Hq,
                                             uint8_t *__restrict__ oq, float *__restrict__ os,
                                             uint16_t *__restrict__ ob) {
  float mx = -INFINITY;
  for (int s = 0; s < used; ++s) mx = fmaxf(mx, wm[bh * S + s]);
  float l = 0.f, a0 = 0.f, a1 = 0.f;
  for (int s = 0; s < used; ++s) {
    const float f = expf(wm[bh * S + s] - mx);
    l = fmaf(f, wl[bh * S + s], l);
    const float *ap = wacc + (bh * S + s) * kHeadDim + 2 * lane;
    a0 = fmaf(f, ap[0], a0);
    a1 = fmaf(f, ap[1], a1);
  }
  a0 /= l;
  a1 /= l;
  if (ob) reinterpret_cast<uint32_t *>(ob)[bh * 64 + lane] = f32_bf16(a0) | (f32_bf16(a1) << 16);
  float amax = wave_max(fmaxf(fabsf(a0), fabsf(a1)));
  const float sc = amax > 0.f ? amax / kFp8Max : 1.f;
  const uint32_t q2 = f32_e4m3(a0 / sc) | (f32_e4m3(a1 / sc) << 8);
  // row b = bh / Hq, group = head: bytes 2 lane, 2 lane + 1 of the group
  const int b = (int)(bh / (size_t)Hq), head = (int)(bh % (size_t)Hq);
  *reinterpret_cast<uint16_t *>(oq + tile_chunk_off(b, head, Hq, lane >> 3) + 2 * (lane & 7)) =
      (uint16_t)q2;
  if (lane == 0) os[bh] = sc;
}

// What the fused form of the split kernel needs besides the caches.
struct AttnFused {
  const uint16_t *qkv;  // [B, (Hq + 2 Hkv) * 128], one new token per sequence
  const uint16_t *qn, *kn;
  float eps;
  const float *cosv, *sinv;
};

// Split-sequence attention for one new token per sequence: workgroup
// (b * Hkv + kh, split) handles positions [split*256, +256) of the L =
// pos[0] + 1 cached ones for the G = Hq / Hkv query heads sharing kv head
// kh.  Scores: one lane per position; softmax partials per head; PV: one
// thread per (head, dim pair).  Partials go to work: m, l [B*Hq, S] and
// acc [B*Hq, S, 128].
//
// kFused: q comes from the projection output through the per-head norm and
// rotary embedding (norm_rope_pair), and the split holding position pos[0]
// first writes the new token's k and v to the caches -- the work of
// qk_norm_rope_kernel, in the same arithmetic.  (Merging the splits in the
// last workgroup to finish would need device-scope fences, which on this
// multi-XCD part write back and invalidate the whole L2: the merge stays a
// kernel of its own.)
template <int G, bool kFused>
__global__ __launch_bounds__(256) void attn_split_kernel(const uint16_t *__restrict__ q,
                                                         uint16_t *__restrict__ kc,
                                                         uint16_t *__restrict__ vc,
                                                         const int *__restrict__ pos, int Hkv,
                                                         int Lmax, int S, float *__restrict__ wm,
                                                         float *__restrict__ wl,
                                                         float *__restrict__ wacc, AttnFused fu) {
  __shared__ float qs[G][kHeadDim];
  __shared__ float pw[G][kAttnChunk];
  __shared__ float part[4 * G * kHeadDim];  // PV partials [wave][head][dim]
  __shared__ float red[G][4];
  const int bk = blockIdx.x, split = blockIdx.y;
  const int b = bk / Hkv, kh = bk % Hkv;
  const int Hq = Hkv * G;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int p = pos[0];
  int L = p + 1;
  L = L < 1 ? 1 : (L > Lmax ? Lmax : L);
  const int c0 = split * kAttnChunk;
  const size_t head0 = (size_t)b * Hq + kh * G;
  if (c0 >= L) {
    if (t < G) {
      wm[(head0 + t) * S + split] = -INFINITY;
      wl[(head0 + t) * S + split] = 0.f;
    }
    return;
  }
  const int n = min(kAttnChunk, L - c0);
  const float scale = rsqrtf((float)kHeadDim);
  if constexpr (kFused) {
    const uint16_t *row = fu.qkv + (size_t)b * (Hq + 2 * Hkv) * kHeadDim;
    const int pc = min(max(p, 0), Lmax - 1);  // rotary row (p is in range for a valid call)
    for (int h = wave; h < G; h += 4) {
      const uint32_t x2 =
          *reinterpret_cast<const uint32_t *>(row + (kh * G + h) * kHeadDim + 2 * lane);
      const uint32_t y2 = norm_rope_pair(x2, fu.qn, fu.eps, fu.cosv, fu.sinv, pc, lane);
      qs[h][2 * lane] = bf16_f32(y2 & 0xffffu) * scale;
      qs[h][2 * lane + 1] = bf16_f32(y2 >> 16) * scale;
    }
    if (p >= c0 && p < c0 + kAttnChunk && p < Lmax && wave < 2) {
      // the new token's k (wave 0) and v (wave 1) go to the caches first
      const int hh = Hq + wave * Hkv + kh;
      const uint32_t x2 = *reinterpret_cast<const uint32_t *>(row + hh * kHeadDim + 2 * lane);
      const uint32_t y2 = wave == 0 ? norm_rope_pair(x2, fu.kn, fu.eps, fu.cosv, fu.sinv, p, lane)
                                    : x2;
      uint16_t *cache = wave == 0 ? kc : vc;
      *reinterpret_cast<uint32_t *>(cache + (((size_t)b * Hkv + kh) * Lmax + p) * kHeadDim +
                                    2 * lane) = y2;
    }
    __threadfence_block();  // the row is read back below by other waves
  } else {
    for (int i = t; i < G * kHeadDim; i += 256) {
      qs[i / kHeadDim][i % kHeadDim] =
          bf16_f32(q[(head0 + i / kHeadDim) * kHeadDim + i % kHeadDim]) * scale;
    }
  }
  __syncthreads();

  const int j = 64 * wave + lane;  // position within the chunk
  float s[G];
#pragma unroll
  for (int h = 0; h < G; ++h) s[h] = 0.f;
  const bool valid = j < n;
  if (valid) {
    // the whole 256-byte key row in flight at once
    const uint4 *kr = reinterpret_cast<const uint4 *>(kc + (((size_t)b * Hkv + kh) * Lmax + c0 + j) * kHeadDim);
    uint4 kv[kHeadDim / 8];
#pragma unroll
    for (int c = 0; c < kHeadDim / 8; ++c) kv[c] = kr[c];
#pragma unroll
    for (int c = 0; c < kHeadDim / 8; ++c) {
      const uint32_t wds[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float k0 = bf16_f32(wds[e] & 0xffffu), k1 = bf16_f32(wds[e] >> 16);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          s[h] = fmaf(qs[h][8 * c + 2 * e], k0, s[h]);
          s[h] = fmaf(qs[h][8 * c + 2 * e + 1], k1, s[h]);
        }
      }
    }
  }
  float mh[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mw = wave_max(valid ? s[h] : -INFINITY);
    if (lane == 0) red[h][wave] = mw;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) mh[h] = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float e = valid ? expf(s[h] - mh[h]) : 0.f;
    pw[h][j] = e;
    const float sw = wave_sum(e);
    if (lane == 0) red[h][wave] = sw;
  }
  __syncthreads();
  if (t < G) {
    wm[(head0 + t) * S + split] = mh[t];
    wl[(head0 + t) * S + split] = (red[t][0] + red[t][1]) + (red[t][2] + red[t][3]);
  }
  // PV: wave w takes positions [64w, 64w + 64) of the chunk, four rows per
  // step (lane / 16), eight dims per lane (16-byte loads), all 16 row loads
  // in flight; positions past n read row n - 1 with weight 0.
  const int dg = lane & 15, rr = lane >> 4;
  const uint16_t *vbase = vc + (((size_t)b * Hkv + kh) * Lmax + c0) * kHeadDim + 8 * dg;
  uint4 vv[16];
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const int jj = min(64 * wave + 4 * st + rr, n - 1);
    vv[st] = *reinterpret_cast<const uint4 *>(vbase + (size_t)jj * kHeadDim);
  }
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const int jp = 64 * wave + 4 * st + rr;
    const uint32_t wds[4] = {vv[st].x, vv[st].y, vv[st].z, vv[st].w};
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p = pw[h][jp];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[h][2 * e] = fmaf(p, bf16_f32(wds[e] & 0xffffu), acc[h][2 * e]);
        acc[h][2 * e + 1] = fmaf(p, bf16_f32(wds[e] >> 16), acc[h][2 * e + 1]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[h][e];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[h][e] = v;
    }
  if (rr == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) part[(wave * G + h) * kHeadDim + 8 * dg + e] = acc[h][e];
  }
  __syncthreads();
  for (int v = t; v < G * kHeadDim; v += 256) {
    const int h = v / kHeadDim, d = v % kHeadDim;
    const float sum = (part[(0 * G + h) * kHeadDim + d] + part[(1 * G + h) * kHeadDim + d]) +
                      (part[(2 * G + h) * kHeadDim + d] + part[(3 * G + h) * kHeadDim + d]);
    wacc[((head0 + h) * S + split) * kHeadDim + d] = sum;
  }
}

// Merge the splits of one (b, head) and quantize the head's 128 outputs
// (one activation group of the o projection); optionally also write bf16.
__global__ __launch_bounds__(64) void attn_combine_kernel(const float *__restrict__ wm,
                                                          const float *__restrict__ wl,
                                                          const float *__restrict__ wacc,
                                                          const int *__restrict__ pos, int Lmax,
                                                          int S, int Hq, uint8_t *__restrict__ oq,
                                                          float *__restrict__ os,
                                                          uint16_t *__restrict__ ob) {
  int L = pos[0] + 1;
  L = L < 1 ? 1 : (L > Lmax ? Lmax : L);
  const int used = (L + kAttnChunk - 1) / kAttnChunk;
  combine_head(wm, wl, wacc, blockIdx.x, S, used, threadIdx.x, Hq, oq, os, ob);
}

// ---------------------------------------------------- FP8 block dequantize

// e4m3fn byte -> fp32 (exact; 0x7F / 0xFF, the NaN codes, become NaN)
__device__ __forceinline__ float e4m3_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  if (e == 0) return __uint_as_float(sign | __float_as_uint((float)m * 0.001953125f));  // m * 2^-9
  if (e == 15 && m == 7) return __uint_as_float(sign | 0x7FC00000u);
  return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

// out[r, c] = bf16(w[r, c] * scale[r / 128, c / 128]); one thread per 16
// consecutive bytes of a row (always inside one 128-column group).
__global__ __launch_bounds__(256) void dequant_fp8_block_kernel(const uint8_t *__restrict__ w,
                                                                const float *__restrict__ scale,
                                                                int64_t n, int64_t k,
                                                                uint16_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte unit
  const int64_t units_per_row = k / 16;
  if (i >= n * units_per_row) return;
  const int64_t r = i / units_per_row, c = (i % units_per_row) * 16;
  const float sc = scale[(r / kGroup) * (k / kGroup) + c / kGroup];
  const uint4 b = *reinterpret_cast<const uint4 *>(w + r * k + c);
  const uint32_t wd[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v0 = e4m3_f32(wd[j] & 0xFFu) * sc, v1 = e4m3_f32((wd[j] >> 8) & 0xFFu) * sc;
    const float v2 = e4m3_f32((wd[j] >> 16) & 0xFFu) * sc, v3 = e4m3_f32(wd[j] >> 24) * sc;
    o[2 * j] = f32_bf16(v0) | (f32_bf16(v1) << 16);
    o[2 * j + 1] = f32_bf16(v2) | (f32_bf16(v3) << 16);
  }
  uint4 *op = reinterpret_cast<uint4 *>(out + r * k + c);
  op[0] = make_uint4(o[0], o[1], o[2], o[3]);
  op[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// ------------------------------------------------------------ MoE routing

// Router logits: logits[m, e] = x[m] . wr[e] over H (bf16 inputs, fp32
// products accumulated per lane in order, then summed across the wave in a
// fixed tree).  Workgroup (ex, tb): wave w takes expert 4 ex + w and tokens
// [4 tb, +4); every load of a 2048-column slice is issued before its FMAs.
// H a multiple of 512.
__global__ __launch_bounds__(256) void moe_logits_kernel(const uint16_t *__restrict__ x,
                                                         const uint16_t *__restrict__ wr, int M,
                                                         int H, int E,
                                                         float *__restrict__ logits) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  const int m0 = blockIdx.y * 4;
  if (e >= E) return;  // uniform per wave; no barrier below
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int h0 = 0; h0 < H; h0 += 2048) {
    uint4 wv[4], xv[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = h0 + 512 * j + 8 * lane;
      const bool in = h0 + 512 * j < H;
      wv[j] = in ? *reinterpret_cast<const uint4 *>(wr + (size_t)e * H + c) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = min(m0 + t, M - 1);  // rows past M re-read row M - 1, unused
        xv[t][j] = in ? *reinterpret_cast<const uint4 *>(x + (size_t)m * H + c)
                      : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t xw[4] = {xv[t][j].x, xv[t][j].y, xv[t][j].z, xv[t][j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[t] = fmaf(bf16_f32(xw[i] & 0xffffu), bf16_f32(ww[i] & 0xffffu), acc[t]);
          acc[t] = fmaf(bf16_f32(xw[i] >> 16), bf16_f32(ww[i] >> 16), acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float v = wave_sum(acc[t]);
    if (lane == 0 && m0 + t < M) logits[(size_t)(m0 + t) * E + e] = v;
  }
}

// Top-k of one token per wave (4 tokens per 256-thread workgroup): softmax
// over the E <= 256 logits in fp32, the top_k largest probabilities (ties
// to the lower expert index), renormalized to sum 1.
__global__ __launch_bounds__(256) void moe_topk_kernel(const float *__restrict__ logits, int M,
                                                       int E, int top_k,
                                                       int *__restrict__ topk_idx,
                                                       float *__restrict__ topk_w) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;  // uniform per wave; no barrier below
  // lane l holds experts l, l + 64, l + 128, l + 192
  float p[4];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    p[i] = e < E ? logits[(size_t)m * E + e] : -INFINITY;
    mx = fmaxf(mx, p[i]);
  }
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = lane + 64 * i < E ? expf(p[i] - mx) : 0.f;
    sum += p[i];
  }
  sum = wave_sum(sum);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = lane + 64 * i < E ? p[i] / sum : -1.f;  // -1: not a choice
  float my_w = 0.f, sel_sum = 0.f;
  int my_i = 0;
  for (int k = 0; k < top_k; ++k) {
    float bv = -2.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (p[i] > bv) {
        bv = p[i];
        bi = lane + 64 * i;
      }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    // every lane now holds the same (bv, bi)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + 64 * i == bi) p[i] = -1.f;
    sel_sum += bv;
    if (lane == k) {
      my_w = bv;
      my_i = bi;
    }
  }
  if (lane < top_k) {
    topk_idx[(size_t)m * top_k + lane] = my_i;
    topk_w[(size_t)m * top_k + lane] = my_w / sel_sum;
  }
}

// Group the P = M * top_k (token, expert) pairs by expert (one workgroup
// of 1024 threads, P <= 8192, E <= 256): pairs of expert e take sorted
// positions [offsets[e], offsets[e + 1]) in token order; pair_tok / pair_w
// give each sorted position's token and routing weight, pair_pos each
// pair's sorted position; active[0, n_active) lists the experts with pairs
// in increasing order; select[e] (optional) = 1 if expert e has pairs.
// Expert ids outside [0, E) are clamped into it.  Two passes over chunks of
// 1024 pairs: integer counts per expert, then each pair's rank = pairs of
// its expert in earlier chunks + earlier pairs of its chunk.
__global__ __launch_bounds__(1024) void moe_group_kernel(
    const int *__restrict__ topk_idx, const float *__restrict__ topk_w, int P, int top_k, int E,
    int *__restrict__ offsets, int *__restrict__ active, int *__restrict__ n_active,
    int *__restrict__ pair_tok, float *__restrict__ pair_w, int *__restrict__ pair_pos,
    int *__restrict__ select) {
  constexpr int kChunk = 1024;
  __shared__ int s_e[kChunk];
  __shared__ int s_cnt[256];
  __shared__ int s_off[257];
  const int t = threadIdx.x;
  auto expert_of = [&](int p) { return p < P ? min(max(topk_idx[p], 0), E - 1) : -1; };
  if (t < 256) s_cnt[t] = 0;
  for (int c0 = 0; c0 < P; c0 += kChunk) {
    const int n = min(kChunk, P - c0);
    __syncthreads();  // s_e of the previous chunk is no longer read
    s_e[t] = expert_of(c0 + t);
    __syncthreads();
    if (t < E) {
      int c = 0;
      for (int q = 0; q < n; ++q) c += s_e[q] == t;
      s_cnt[t] += c;
    }
  }
  __syncthreads();
  if (t < 64) {
    // wave 0: exclusive prefix of the counts and of the active flags over
    // E <= 256 experts, 4 consecutive experts per lane
    int c[4], f[4], sc = 0, sf = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * t + i;
      c[i] = e < E ? s_cnt[e] : 0;
      f[i] = c[i] > 0;
      sc += c[i];
      sf += f[i];
    }
    int ic = sc, jf = sf;  // inclusive scans across lanes
    for (int o = 1; o < 64; o <<= 1) {
      const int uc = __shfl_up(ic, o), uf = __shfl_up(jf, o);
      if (t >= o) {
        ic += uc;
        jf += uf;
      }
    }
    int off = ic - sc, na = jf - sf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * t + i;
      if (e < E) {
        s_off[e] = off;
        if (f[i]) active[na] = e;
      }
      off += c[i];
      na += f[i];
    }
    if (t == 63) {
      s_off[E] = ic;
      *n_active = jf;
    }
  }
  __syncthreads();
  for (int i = t; i <= E; i += kChunk) offsets[i] = s_off[i];
  if (select && t < E) select[t] = s_cnt[t] > 0 ? 1 : 0;
  __syncthreads();
  if (t < 256) s_cnt[t] = 0;  // now: pairs of each expert in earlier chunks
  for (int c0 = 0; c0 < P; c0 += kChunk) {
    const int n = min(kChunk, P - c0);
    __syncthreads();
    const int e = expert_of(c0 + t);
    s_e[t] = e;
    __syncthreads();
    if (t < n) {
      int rank = s_cnt[e];
      for (int q = 0; q < t; ++q) rank += s_e[q] == e;
      const int q = s_off[e] + rank;
      pair_tok[q] = (c0 + t) / top_k;
      pair_w[q] = topk_w[c0 + t];
      pair_pos[c0 + t] = q;
    }
    __syncthreads();  // every rank read s_cnt before it grows
    if (t < E) {
      int c = 0;
      for (int q = 0; q < n; ++q) c += s_e[q] == t;
      s_cnt[t] += c;
    }
  }
}

// Grouped small-M FP8 linear over the active experts: workgroup (tile,
// slot) computes output columns [16 tile, +16) of expert e = active[slot]
// for its rows [offsets[e], offsets[e + 1]) in chunks of 16:
//   out[q, col] = sum_g (sum_{k in g} aq[row(q), k] * w_e[n, k]) * as[row(q), g] * ws_e[n/128, g]
// with row(q) = row_of[q] (a gather, e.g. the token of a sorted pair) or q.
// Segment s of an expert (e.g. gate, up) owns output columns
// [s * seg_n, +seg_n).  Slots past n_active exit at once, so the grid can
// be sized for every expert and captured in a graph.
struct MoeLinear {
  const uint8_t *aq;
  const float *as;
  const int *row_of;
  const int *offsets;
  const int *active;
  const int *n_active;
  const uint64_t *w;   // [E * n_segs] weight addresses
  const uint64_t *ws;  // [E * n_segs] scale addresses
  uint16_t *out;
  int n_segs, seg_n, K, ldo;
  int wtiled;  // expert weights in the tile layout (else row-major)
};

template <int WAVES, int kU>
__global__ __launch_bounds__(WAVES * 64) void moe_linear16_kernel(MoeLinear a) {
  __shared__ float red[WAVES][4][64];
  const int slot = blockIdx.y;
  if (slot >= a.n_active[0]) return;  // uniform
  const int e = a.active[slot];
  const int r0 = a.offsets[e], rows = a.offsets[e + 1] - r0;
  const int seg = (int)(blockIdx.x * 16) / a.seg_n;
  const int n0 = (int)(blockIdx.x * 16) - seg * a.seg_n;
  const uint8_t *w = reinterpret_cast<const uint8_t *>(a.w[(size_t)e * a.n_segs + seg]);
  const float *ws = reinterpret_cast<const float *>(a.ws[(size_t)e * a.n_segs + seg]);
  const int col = seg * a.seg_n;
  const int K = a.K, kgroups = K / kGroup;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const WeightLane wl(w, a.wtiled != 0, n0, r, g, K);
  const Rsrc wr = wl.rsrc(K);
  const float *wsrow = ws + (size_t)(n0 / kGroup) * kgroups;

  for (int rc = 0; rc < rows; rc += 16) {
    const int mrows = min(16, rows - rc);
    const bool row_ok = r < mrows;
    const int q = r0 + rc + (row_ok ? r : 0);
    const uint8_t *arow = tile_lane_base(a.aq, a.row_of ? a.row_of[q] : q, kgroups, g);
    bool srow_ok[4];
    const float *srow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      srow_ok[i] = 4 * g + i < mrows;
      const int qi = r0 + rc + (srow_ok[i] ? 4 * g + i : 0);
      srow[i] = a.as + (size_t)(a.row_of ? a.row_of[qi] : qi) * kgroups;
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int kb = wave; kb < kgroups; kb += WAVES * kU) {
      uint4 wv[kU][2], av[kU][2];
      float wsv[kU], sav[kU][4];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int kg = kb + WAVES * u;
        if (kg < kgroups) {
          wl.load(wr, kg, wv[u][0], wv[u][1]);
          wsv[u] = wsrow[kg];
          av[u][0] = *reinterpret_cast<const uint4 *>(arow + (size_t)kg * 2048);
          av[u][1] = *reinterpret_cast<const uint4 *>(arow + (size_t)kg * 2048 + 1024);
#pragma unroll
          for (int i = 0; i < 4; ++i) sav[u][i] = srow[i][kg];
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int kg = kb + WAVES * u;
        if (kg >= kgroups) break;
        if (!row_ok) av[u][0] = av[u][1] = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sav[u][i] = srow_ok[i] ? sav[u][i] : 0.f;
        v4f d = {0.f, 0.f, 0.f, 0.f};
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av[u][0].y << 32) | av[u][0].x),
            (long)(((uint64_t)wv[u][0].y << 32) | wv[u][0].x), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av[u][0].w << 32) | av[u][0].z),
            (long)(((uint64_t)wv[u][0].w << 32) | wv[u][0].z), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av[u][1].y << 32) | av[u][1].x),
            (long)(((uint64_t)wv[u][1].y << 32) | wv[u][1].x), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            (long)(((uint64_t)av[u][1].w << 32) | av[u][1].z),
            (long)(((uint64_t)wv[u][1].w << 32) | wv[u][1].z), d, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], sav[u][i] * wsv[u], acc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    // the 256 sums (4 accumulators x 64 lanes), over the threads
    for (int t = threadIdx.x; t < 256; t += WAVES * 64) {
      const int i = t >> 6, l = t & 63;
      float sum = 0.f;
#pragma unroll
      for (int wv2 = 0; wv2 < WAVES; ++wv2) sum += red[wv2][i][l];
      const int m = 4 * (l >> 4) + i;
      if (m < mrows)
        a.out[(size_t)(r0 + rc + m) * a.ldo + col + n0 + (l & 15)] = (uint16_t)f32_bf16(sum);
    }
    __syncthreads();  // red is rewritten by the next chunk
  }
}

// y[m, :] = sum_k pair_w[q] * down[q, :] over q = pair_pos[m * top_k + k],
// k = 0 .. top_k - 1 in order, accumulated in fp32; bf16 out [M, H].  One
// workgroup per token, 8 columns per thread.
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t *__restrict__ down,
                                                          int ldd, const int *__restrict__ pair_pos,
                                                          const float *__restrict__ pair_w,
                                                          int top_k, int H,
                                                          uint16_t *__restrict__ out) {
  const int m = blockIdx.x;
  for (int c = 8 * threadIdx.x; c < H; c += 8 * 256) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < top_k; ++k) {
      const int q = pair_pos[(size_t)m * top_k + k];
      const float wq = pair_w[q];
      const uint4 v = *reinterpret_cast<const uint4 *>(down + (size_t)q * ldd + c);
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(wq, bf16_f32(wd[i] & 0xffffu), acc[2 * i]);
        acc[2 * i + 1] = fmaf(wq, bf16_f32(wd[i] >> 16), acc[2 * i + 1]);
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32_bf16(acc[2 * i]) | (f32_bf16(acc[2 * i + 1]) << 16);
    *reinterpret_cast<uint4 *>(out + (size_t)m * H + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
inline int launched() { return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP; }

}  // namespace

extern "C" int ecf8_fp8_linear(const void *aq, const float *as, int64_t M, int64_t K,
                               const ecf8_linear_seg *segs, int n_segs, void *out, int64_t ldo,
                               void *stream) {
  if (!aq || !as || !segs || !out || M <= 0 || K <= 0 || n_segs < 1 ||
      n_segs > ECF8_LINEAR_MAX_SEGS)
    return ECF8_ERR_INVALID_ARG;
  if (K % kGroup || M > (1 << 24) || K > (1 << 20)) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(aq, 16) || !aligned(out, 4) || !aligned(as, 4)) return ECF8_ERR_MISALIGNED;
  LinearSegs s{};
  int64_t n_total = 0;
  for (int i = 0; i < n_segs; ++i) {
    const ecf8_linear_seg &g = segs[i];
    if (!g.weight || !g.weight_scale || g.n <= 0 || g.out_col < 0) return ECF8_ERR_INVALID_ARG;
    if (g.weight_layout != ECF8_WEIGHT_ROWS && g.weight_layout != ECF8_WEIGHT_TILES)
      return ECF8_ERR_INVALID_ARG;
    if (g.n % kGroup) return ECF8_ERR_UNSUPPORTED;
    if (!aligned(g.weight, 16) || !aligned(g.weight_scale, 4)) return ECF8_ERR_MISALIGNED;
    if (g.out_col + g.n > ldo) return ECF8_ERR_CAPACITY;
    n_total += g.n;
    s.w[i] = static_cast<const uint8_t *>(g.weight);
    s.ws[i] = g.weight_scale;
    s.n_end[i] = (int)n_total;
    s.col[i] = (int)g.out_col;
    s.tiled[i] = g.weight_layout == ECF8_WEIGHT_TILES;
  }
  if (n_total > (1 << 24)) return ECF8_ERR_UNSUPPORTED;
  s.count = n_segs;
  const auto *a = static_cast<const uint8_t *>(aq);
  auto *o = static_cast<uint16_t *>(out);
  if (M <= 16) {
    const unsigned n_tiles = (unsigned)(n_total / 16);
    int dev = 0, cus = 0;
    // more tiles than two workgroups per CU at K = 4096: the persistent form
    if (K == 4096 && hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n_tiles > 2u * (unsigned)cus) {
      fp8_linear16p_kernel<16><<<(unsigned)cus, 1024, 0, as_stream(stream)>>>(
          a, as, (int)M, s, o, (int)ldo, (int)n_tiles);
      return launched();
    }
    // long K: 16 waves, so each wave's share stays within two batches;
    // at most one tile per CU: 16 waves, so the fused linear summing in the
    // same order runs 16 waves per CU (Qwen3-8B o projection: fused 9.8 ->
    // 8.4 us, FP8 unchanged at 5.5)
    if (K / kGroup >= 64 ||
        (hipGetDevice(&dev) == hipSuccess &&
         hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
         n_tiles <= (unsigned)cus))
      fp8_linear16_kernel<16><<<n_tiles, 1024, 0, as_stream(stream)>>>(a, as, (int)M, (int)K, s,
                                                                       o, (int)ldo);
    else
      fp8_linear16_kernel<8><<<n_tiles, 512, 0, as_stream(stream)>>>(a, as, (int)M, (int)K, s, o,
                                                                     (int)ldo);
  } else {
    const int n_mb = (int)((M + kGemmBM - 1) / kGemmBM);
    const int64_t n_tiles = (n_total / kGemmBN) * n_mb;
    if (n_tiles > INT32_MAX) return ECF8_ERR_UNSUPPORTED;
    fp8_gemm_kernel<<<(unsigned)n_tiles, kGemmWaves * 64, 0, as_stream(stream)>>>(
        a, as, (int)M, (int)K, s, o, (int)ldo, n_mb, (int)n_tiles);
  }
  return launched();
}

extern "C" int ecf8_rmsnorm(const void *x, float *residual, const void *weight, float eps, int64_t M,
                            int64_t K, void *out_q, float *out_scale, void *out_bf16, void *stream) {
  if (!residual || !weight || M <= 0 || (!out_bf16 && !out_q) || (!out_q != !out_scale))
    return ECF8_ERR_INVALID_ARG;
  if ((K != 4096 && K != 2048) || M > 0x7fffffff) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(residual, 16) || (x && !aligned(x, 16)) || !aligned(weight, 16) ||
      (out_q && !aligned(out_q, 16)) || (out_bf16 && !aligned(out_bf16, 16)))
    return ECF8_ERR_MISALIGNED;
  const auto *xp = static_cast<const uint16_t *>(x);
  const auto *wp = static_cast<const uint16_t *>(weight);
  auto *qp = static_cast<uint8_t *>(out_q);
  auto *bp = static_cast<uint16_t *>(out_bf16);
  if (K == 4096)
    rmsnorm_kernel<256><<<(unsigned)M, 256, 0, as_stream(stream)>>>(xp, residual, wp, eps, (int)K,
                                                                    qp, out_scale, bp);
  else
    rmsnorm_kernel<128><<<(unsigned)M, 128, 0, as_stream(stream)>>>(xp, residual, wp, eps, (int)K,
                                                                    qp, out_scale, bp);
  return launched();
}

extern "C" int ecf8_silu_mul_quant(const void *gate_up, int64_t M, int64_t I, void *out_q,
                                   float *out_scale, void *stream) {
  if (!gate_up || !out_q || !out_scale || M <= 0 || I <= 0) return ECF8_ERR_INVALID_ARG;
  if (I % kGroup || I > (1 << 24) || M > 65535) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(gate_up, 16) || !aligned(out_q, 16)) return ECF8_ERR_MISALIGNED;
  silu_mul_quant_kernel<<<dim3((unsigned)((I + 4095) / 4096), (unsigned)M), 256, 0,
                          as_stream(stream)>>>(
      static_cast<const uint16_t *>(gate_up), (int)I, static_cast<uint8_t *>(out_q), out_scale);
  return launched();
}

extern "C" int ecf8_act_quant(const void *x, int64_t M, int64_t K, void *out_q, float *out_scale,
                              void *stream) {
  if (!x || !out_q || !out_scale || M <= 0 || K <= 0) return ECF8_ERR_INVALID_ARG;
  if (K % kGroup || K > (1 << 24) || M > 65535) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(x, 16) || !aligned(out_q, 16)) return ECF8_ERR_MISALIGNED;
  act_quant_kernel<<<dim3((unsigned)((K + 4095) / 4096), (unsigned)M), 256, 0,
                     as_stream(stream)>>>(
      static_cast<const uint16_t *>(x), (int)K, static_cast<uint8_t *>(out_q), out_scale);
  return launched();
}

extern "C" int ecf8_qk_norm_rope(const void *qkv, int64_t B, int64_t T, int Hq, int Hkv,
                                 const void *q_norm, const void *k_norm, float eps, const float *cos_t,
                                 const float *sin_t, const int *pos, int64_t Lmax, void *q_out,
                                 void *k_cache, void *v_cache, void *stream) {
  if (!qkv || !q_norm || !k_norm || !cos_t || !sin_t || !pos || !q_out || !k_cache || !v_cache ||
      B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Lmax <= 0)
    return ECF8_ERR_INVALID_ARG;
  const int64_t items = B * T * (Hq + 2 * Hkv);
  if (items > (int64_t)1 << 30) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(qkv, 4) || !aligned(q_norm, 4) || !aligned(k_norm, 4) || !aligned(q_out, 4) ||
      !aligned(k_cache, 4) || !aligned(v_cache, 4))
    return ECF8_ERR_MISALIGNED;
  qk_norm_rope_kernel<<<(unsigned)((items + 3) / 4), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t *>(qkv), (int)T, Hq, Hkv, static_cast<const uint16_t *>(q_norm),
      static_cast<const uint16_t *>(k_norm), eps, cos_t, sin_t, pos, (int)Lmax,
      static_cast<uint16_t *>(q_out), static_cast<uint16_t *>(k_cache),
      static_cast<uint16_t *>(v_cache), (int)items);
  return launched();
}

extern "C" int ecf8_dequant_fp8_block(const void *weight, const float *weight_scale, int64_t n,
                                      int64_t k, void *out, void *stream) {
  if (!weight || !weight_scale || !out || n <= 0 || k <= 0) return ECF8_ERR_INVALID_ARG;
  if (n % kGroup || k % kGroup || n * k > ((int64_t)1 << 40)) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(weight, 16) || !aligned(out, 16) || !aligned(weight_scale, 4))
    return ECF8_ERR_MISALIGNED;
  const int64_t units = n * (k / 16);
  dequant_fp8_block_kernel<<<(unsigned)((units + 255) / 256), 256, 0, as_stream(stream)>>>(
      static_cast<const uint8_t *>(weight), weight_scale, n, k, static_cast<uint16_t *>(out));
  return launched();
}

extern "C" int64_t ecf8_attention_work_floats(int64_t B, int Hq, int64_t Lmax) {
  if (B <= 0 || Hq <= 0 || Lmax <= 0) return -1;
  const int64_t S = (Lmax + kAttnChunk - 1) / kAttnChunk;
  return B * Hq * S * (kHeadDim + 2);
}

extern "C" int ecf8_decode_attention(const void *q, const void *k_cache, const void *v_cache,
                                     const int *pos, int64_t B, int Hq, int Hkv, int64_t Lmax,
                                     float *work, int64_t work_floats, void *out_q,
                                     float *out_scale, void *out_bf16, void *stream) {
  if (!q || !k_cache || !v_cache || !pos || !work || !out_q || !out_scale || B <= 0 || Hq <= 0 ||
      Hkv <= 0 || Lmax <= 0)
    return ECF8_ERR_INVALID_ARG;
  if ((Hq != 4 * Hkv && Hq != 8 * Hkv) || B * Hkv > 65535 || Lmax > (1 << 24))
    return ECF8_ERR_UNSUPPORTED;
  const int64_t S = (Lmax + kAttnChunk - 1) / kAttnChunk;
  if (work_floats < B * Hq * S * (kHeadDim + 2)) return ECF8_ERR_CAPACITY;
  if (!aligned(q, 4) || !aligned(k_cache, 16) || !aligned(v_cache, 4) || !aligned(work, 8) ||
      !aligned(out_q, 2) || (out_bf16 && !aligned(out_bf16, 4)))
    return ECF8_ERR_MISALIGNED;
  float *wm = work, *wl = work + B * Hq * S, *wacc = work + 2 * B * Hq * S;
  const dim3 grid((unsigned)(B * Hkv), (unsigned)S);
  const auto *qp = static_cast<const uint16_t *>(q);
  auto *kp = static_cast<uint16_t *>(const_cast<void *>(k_cache));
  auto *vp = static_cast<uint16_t *>(const_cast<void *>(v_cache));
  const AttnFused none{};
  if (Hq == 4 * Hkv)
    attn_split_kernel<4, false><<<grid, 256, 0, as_stream(stream)>>>(
        qp, kp, vp, pos, Hkv, (int)Lmax, (int)S, wm, wl, wacc, none);
  else
    attn_split_kernel<8, false><<<grid, 256, 0, as_stream(stream)>>>(
        qp, kp, vp, pos, Hkv, (int)Lmax, (int)S, wm, wl, wacc, none);
  attn_combine_kernel<<<(unsigned)(B * Hq), 64, 0, as_stream(stream)>>>(
      wm, wl, wacc, pos, (int)Lmax, (int)S, Hq, static_cast<uint8_t *>(out_q), out_scale,
      static_cast<uint16_t *>(out_bf16));
  return launched();
}

extern "C" int ecf8_decode_attention_fused(const void *qkv, int64_t B, int Hq, int Hkv,
                                           const void *q_norm, const void *k_norm, float eps,
                                           const float *cos_t, const float *sin_t, const int *pos,
                                           int64_t Lmax, void *k_cache, void *v_cache,
                                           float *work, int64_t work_floats, void *out_q,
                                           float *out_scale, void *out_bf16, void *stream) {
  if (!qkv || !q_norm || !k_norm || !cos_t || !sin_t || !pos || !k_cache || !v_cache || !work ||
      !out_q || !out_scale || B <= 0 || Hq <= 0 || Hkv <= 0 || Lmax <= 0)
    return ECF8_ERR_INVALID_ARG;
  if ((Hq != 4 * Hkv && Hq != 8 * Hkv) || B * Hkv > 65535 || Lmax > (1 << 24))
    return ECF8_ERR_UNSUPPORTED;
  const int64_t S = (Lmax + kAttnChunk - 1) / kAttnChunk;
  if (work_floats < B * Hq * S * (kHeadDim + 2)) return ECF8_ERR_CAPACITY;
  if (!aligned(qkv, 4) || !aligned(q_norm, 4) || !aligned(k_norm, 4) || !aligned(k_cache, 16) ||
      !aligned(v_cache, 4) || !aligned(work, 8) || !aligned(out_q, 2) ||
      (out_bf16 && !aligned(out_bf16, 4)))
    return ECF8_ERR_MISALIGNED;
  float *wm = work, *wl = work + B * Hq * S, *wacc = work + 2 * B * Hq * S;
  const AttnFused fu{static_cast<const uint16_t *>(qkv), static_cast<const uint16_t *>(q_norm),
                     static_cast<const uint16_t *>(k_norm), eps, cos_t, sin_t};
  const dim3 grid((unsigned)(B * Hkv), (unsigned)S);
  auto *kp = static_cast<uint16_t *>(k_cache);
  auto *vp = static_cast<uint16_t *>(v_cache);
  if (Hq == 4 * Hkv)
    attn_split_kernel<4, true><<<grid, 256, 0, as_stream(stream)>>>(
        nullptr, kp, vp, pos, Hkv, (int)Lmax, (int)S, wm, wl, wacc, fu);
  else
    attn_split_kernel<8, true><<<grid, 256, 0, as_stream(stream)>>>(
        nullptr, kp, vp, pos, Hkv, (int)Lmax, (int)S, wm, wl, wacc, fu);
  attn_combine_kernel<<<(unsigned)(B * Hq), 64, 0, as_stream(stream)>>>(
      wm, wl, wacc, pos, (int)Lmax, (int)S, Hq, static_cast<uint8_t *>(out_q), out_scale,
      static_cast<uint16_t *>(out_bf16));
  return launched();
}

extern "C" int ecf8_moe_route(const void *x, const void *router_w, int64_t M, int64_t H, int E,
                              int top_k, float *logits, int *topk_idx, float *topk_w,
                              void *stream) {
  if (!x || !router_w || !logits || !topk_idx || !topk_w || M <= 0 || H <= 0 || E <= 0 ||
      top_k <= 0)
    return ECF8_ERR_INVALID_ARG;
  if (H % 512 || H > (1 << 20) || E > 256 || top_k > 16 || top_k > E || M > (1 << 16))
    return ECF8_ERR_UNSUPPORTED;
  if (!aligned(x, 16) || !aligned(router_w, 16) || !aligned(logits, 4) || !aligned(topk_idx, 4) ||
      !aligned(topk_w, 4))
    return ECF8_ERR_MISALIGNED;
  moe_logits_kernel<<<dim3((unsigned)((E + 3) / 4), (unsigned)((M + 3) / 4)), 256, 0,
                      as_stream(stream)>>>(static_cast<const uint16_t *>(x),
                                           static_cast<const uint16_t *>(router_w), (int)M,
                                           (int)H, E, logits);
  moe_topk_kernel<<<(unsigned)((M + 3) / 4), 256, 0, as_stream(stream)>>>(logits, (int)M, E,
                                                                          top_k, topk_idx, topk_w);
  return launched();
}

extern "C" int ecf8_moe_group(const int *topk_idx, const float *topk_w, int64_t M, int top_k, int E,
                              int *offsets, int *active, int *n_active, int *pair_tok,
                              float *pair_w, int *pair_pos, int *select, void *stream) {
  if (!topk_idx || !topk_w || !offsets || !active || !n_active || !pair_tok || !pair_w ||
      !pair_pos || M <= 0 || top_k <= 0 || E <= 0)
    return ECF8_ERR_INVALID_ARG;
  if (M * top_k > 8192 || E > 256) return ECF8_ERR_UNSUPPORTED;
  moe_group_kernel<<<1, 1024, 0, as_stream(stream)>>>(topk_idx, topk_w, (int)(M * top_k), top_k, E,
                                                     offsets, active, n_active, pair_tok, pair_w,
                                                     pair_pos, select);
  return launched();
}

extern "C" int ecf8_moe_linear(const void *aq, const float *as, const int *row_of,
                               const int *offsets, const int *active, const int *n_active,
                               int n_experts, const void *const *weights,
                               const float *const *weight_scales, int n_segs, int64_t seg_n,
                               int64_t K, int weight_layout, void *out, int64_t ldo,
                               void *stream) {
  if (!aq || !as || !offsets || !active || !n_active || !weights || !weight_scales || !out ||
      n_experts <= 0 || n_segs < 1 || n_segs > ECF8_LINEAR_MAX_SEGS || seg_n <= 0 || K <= 0 ||
      (weight_layout != ECF8_WEIGHT_ROWS && weight_layout != ECF8_WEIGHT_TILES))
    return ECF8_ERR_INVALID_ARG;
  if (seg_n % kGroup || K % kGroup || K > (1 << 20) || n_segs * seg_n > (1 << 20) ||
      n_experts > 65535)
    return ECF8_ERR_UNSUPPORTED;
  if (ldo < n_segs * seg_n) return ECF8_ERR_CAPACITY;
  if (!aligned(aq, 16) || !aligned(as, 4) || !aligned(out, 4) || !aligned(weights, 8) ||
      !aligned(weight_scales, 8))
    return ECF8_ERR_MISALIGNED;
  MoeLinear a{static_cast<const uint8_t *>(aq), as, row_of, offsets, active, n_active,
              reinterpret_cast<const uint64_t *>(weights),
              reinterpret_cast<const uint64_t *>(weight_scales), static_cast<uint16_t *>(out),
              n_segs, (int)seg_n, (int)K, (int)ldo, weight_layout == ECF8_WEIGHT_TILES};
  const dim3 grid((unsigned)(n_segs * seg_n / 16), (unsigned)n_experts);
  // each wave's share of the K groups in one batch of loads where it fits.
  // On MI355X, Qwen3-30B-A3B experts at 16 tokens (48 layers back to back):
  // gate/up (K = 2048) 48.5 us per layer at four waves of four groups
  // against 53.4 at eight of two; down (K = 768) 23.7 us at three waves of
  // two groups against 26.9 at four (two, two, one, one)
  const int64_t kg = K / kGroup;
  static_assert(ECF8_MOE_FOUR_WAVE_GROUPS == 16, "four waves of at most four groups");
  if (kg == 6)
    moe_linear16_kernel<3, 2><<<grid, 192, 0, as_stream(stream)>>>(a);
  else if (kg <= 8)
    moe_linear16_kernel<4, 2><<<grid, 256, 0, as_stream(stream)>>>(a);
  else if (kg <= ECF8_MOE_FOUR_WAVE_GROUPS)
    moe_linear16_kernel<4, 4><<<grid, 256, 0, as_stream(stream)>>>(a);
  else
    moe_linear16_kernel<8, 4><<<grid, 512, 0, as_stream(stream)>>>(a);
  return launched();
}

extern "C" int ecf8_moe_combine(const void *down, int64_t ldd, const int *pair_pos,
                                const float *pair_w, int64_t M, int top_k, int64_t H, void *out,
                                void *stream) {
  if (!down || !pair_pos || !pair_w || !out || M <= 0 || top_k <= 0 || H <= 0 || ldd < H)
    return ECF8_ERR_INVALID_ARG;
  if (H % 8 || ldd % 8 || M > 0x7fffffff) return ECF8_ERR_UNSUPPORTED;
  if (!aligned(down, 16) || !aligned(out, 16)) return ECF8_ERR_MISALIGNED;
  moe_combine_kernel<<<(unsigned)M, 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t *>(down), (int)ldd, pair_pos, pair_w, top_k, (int)H,
      static_cast<uint16_t *>(out));
  return launched();
}
