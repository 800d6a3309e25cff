// Streaming kernels for measuring what MI355X sustains (bench.py --mode
// ceiling): a read-only sweep and a copy over a buffer, with the grid, the
// workgroup size, the 16-byte loads each lane keeps in flight and the
// non-temporal hint as parameters.  They bound what a one-launch,
// HBM-streaming kernel of a given size can reach -- the decode and the
// decode-step linears are measured against them.  No reference
// counterpart; nothing on the decode path calls them.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ecf8.h"

namespace {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

template <int V, bool NT>
__device__ __forceinline__ void load_v(const v4u *__restrict__ src, int64_t i, int64_t stride,
                                       v4u (&v)[V]) {
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const v4u *p = src + i + j * stride;
    v[j] = NT ? __builtin_nontemporal_load(p) : *p;
  }
}

// Grid-stride sweep over n16 16-byte words: each lane keeps V loads in
// flight per iteration.  The XOR of everything read is stored only if it
// equals `magic`, which keeps every load without writing anything else.
template <int V, bool NT>
__global__ __launch_bounds__(1024) void stream_read_kernel(const v4u *__restrict__ src,
                                                           int64_t n16, uint32_t magic,
                                                           uint32_t *__restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (V - 1) * stride < n16; i += V * stride) {
    v4u v[V];
    load_v<V, NT>(src, i, stride, v);
#pragma unroll
    for (int j = 0; j < V; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  for (; i < n16; i += stride) {
    const v4u v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == magic) sink[0] = acc;
}

template <int V, bool NT>
__global__ __launch_bounds__(1024) void stream_copy_kernel(const v4u *__restrict__ src,
                                                           v4u *__restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (V - 1) * stride < n16; i += V * stride) {
    v4u v[V];
    load_v<V, NT>(src, i, stride, v);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      v4u *p = dst + i + j * stride;
      if (NT)
        __builtin_nontemporal_store(v[j], p);
      else
        *p = v[j];
    }
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

template <int V, bool NT>
int launch(int op, const void *src, void *dst, int64_t n16, int grid, int block, uint32_t *sink,
           hipStream_t s) {
  const auto *in = static_cast<const v4u *>(src);
  if (op == 0)
    stream_read_kernel<V, NT><<<grid, block, 0, s>>>(in, n16, 0x9E3779B9u, sink);
  else
    stream_copy_kernel<V, NT><<<grid, block, 0, s>>>(in, static_cast<v4u *>(dst), n16);
  return hipGetLastError() == hipSuccess ? ECF8_OK : ECF8_ERR_HIP;
}

template <bool NT>
int by_depth(int depth, int op, const void *src, void *dst, int64_t n16, int grid, int block,
             uint32_t *sink, hipStream_t s) {
  switch (depth) {
    case 1: return launch<1, NT>(op, src, dst, n16, grid, block, sink, s);
    case 2: return launch<2, NT>(op, src, dst, n16, grid, block, sink, s);
    case 4: return launch<4, NT>(op, src, dst, n16, grid, block, sink, s);
    case 8: return launch<8, NT>(op, src, dst, n16, grid, block, sink, s);
    default: return ECF8_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" int ecf8_stream_probe(int op, const void *src, void *dst, int64_t bytes, int grid,
                                 int block, int depth, int nontemporal, uint32_t *sink,
                                 void *stream) {
  if (!src || !sink || bytes <= 0 || grid <= 0 || (op != 0 && op != 1) || (op == 1 && !dst))
    return ECF8_ERR_INVALID_ARG;
  if (block != 64 && block != 128 && block != 256 && block != 512 && block != 1024)
    return ECF8_ERR_UNSUPPORTED;
  if (bytes % 16 || ((uintptr_t)src & 15) || (dst && ((uintptr_t)dst & 15)) ||
      ((uintptr_t)sink & 3))
    return ECF8_ERR_MISALIGNED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return nontemporal ? by_depth<true>(depth, op, src, dst, bytes / 16, grid, block, sink, s)
                     : by_depth<false>(depth, op, src, dst, bytes / 16, grid, block, sink, s);
}
