// fk_misc.h — small kernels the runtime side needs: a fill (graphs clear
// memory with a kernel, never a memset node) and an empty kernel that
// measures what a launch costs.
#pragma once

#include "fk_common.h"

extern "C" __global__ void __launch_bounds__(256) fk_fill_u32(uint32_t *__restrict__ dst, fk_fill_params p) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < p.count; i += gridDim.x * blockDim.x) dst[i] = p.value;
}

extern "C" __global__ void __launch_bounds__(1024) fk_noop(fk_noop_params) {}

// Reads a buffer once, 16 bytes a lane, grid-strided, and stores one word a
// threadgroup: the attainable HBM read bandwidth, the ceiling the
// bandwidth-bound kernels are measured against.
extern "C" __global__ void __launch_bounds__(256)
    fk_stream_read(const uint4 *__restrict__ src, uint32_t *__restrict__ out, fk_stream_read_params p) {
  uint32_t acc = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < p.words; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < p.words; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  for (int m = 1; m < FK_WAVE; m <<= 1) acc ^= __shfl_xor(acc, m);
  if ((threadIdx.x & (FK_WAVE - 1)) == 0) out[blockIdx.x * (blockDim.x / FK_WAVE) + threadIdx.x / FK_WAVE] = acc;
}
