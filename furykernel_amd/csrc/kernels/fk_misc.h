// fk_misc.h — small kernels the runtime side needs: a fill (graphs clear
// memory with a kernel, never a memset node) and an empty kernel that
// measures what a launch costs.
#pragma once

#include "fk_common.h"

struct fk_fill_params {
  uint32_t count;  // 32-bit words
  uint32_t value;
};

extern "C" __global__ void __launch_bounds__(256) fk_fill_u32(uint32_t *__restrict__ dst, fk_fill_params p) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < p.count; i += gridDim.x * blockDim.x) dst[i] = p.value;
}

struct fk_noop_params {
  uint32_t unused;
};

extern "C" __global__ void __launch_bounds__(1024) fk_noop(fk_noop_params) {}
