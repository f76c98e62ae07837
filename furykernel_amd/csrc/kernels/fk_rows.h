// fk_rows.h — reductions over rows: RMSNorm and softmax, one threadgroup per
// row (or segment), in the orders of test/Test/FuryKernel/Kernels.hs:53-74 and
// src/FuryKernel/Reduce.hs:29-85, with packs of four f32 (one 16-byte load).
//
// Thread t visits packs t, t + T, ... of its row; its own sum of squares (or
// maximum, or sum of exps) goes element by element in that order, then
// block_reduce combines the threads.  The orders depend on T, the wavefront
// width and the pack only, so a row's result depends on nothing else in the
// batch.
#pragma once

#include "fk_common.h"

struct fk_rmsnorm_params {
  uint32_t rows;    // rows of x
  uint32_t width;   // elements per row
  uint32_t seg;     // elements per segment (a multiple of 4 dividing width)
  float eps;        // rounded once to binary32
  float factor;     // a constant factor; 1 multiplies by nothing
  uint32_t has_gamma;
};

// One threadgroup per segment: y = ((x * rsqrt(sum x^2 / seg + eps)) * gamma) * factor.
extern "C" __global__ void __launch_bounds__(1024)
    fk_rmsnorm_f32(const float *__restrict__ x, const float *__restrict__ gamma, float *__restrict__ y,
                   fk_rmsnorm_params p) {
  __shared__ float slots[16];
  const uint32_t segs = p.width / p.seg;
  const uint32_t row = blockIdx.x / segs;
  const uint32_t s = blockIdx.x % segs;
  if (row >= p.rows) return;  // uniform across the threadgroup
  const float *xs = x + (size_t)row * p.width + (size_t)s * p.seg;
  float *ys = y + (size_t)row * p.width + (size_t)s * p.seg;
  const uint32_t packs = p.seg / 4;
  float acc = 0.0f;
  for (uint32_t j = threadIdx.x; j < packs; j += blockDim.x) {
    float4 v = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)j);
    acc = acc + v.x * v.x;
    acc = acc + v.y * v.y;
    acc = acc + v.z * v.z;
    acc = acc + v.w * v.w;
  }
  const float total = fk::block_reduce<false>(acc, slots);
  const float scale = fk::rsqrt_once(total / (float)p.seg + p.eps);
  for (uint32_t j = threadIdx.x; j < packs; j += blockDim.x) {
    float4 v = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)j);
    float o[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
    if (p.has_gamma) {
      float4 g = *reinterpret_cast<const float4 *>(gamma + 4 * (size_t)j);
      o[0] = o[0] * g.x;
      o[1] = o[1] * g.y;
      o[2] = o[2] * g.z;
      o[3] = o[3] * g.w;
    }
    if (p.factor != 1.0f) {
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = o[e] * p.factor;
    }
    *reinterpret_cast<float4 *>(ys + 4 * (size_t)j) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

struct fk_softmax_params {
  uint32_t rows;
  uint32_t n;  // elements per row, a multiple of 4
};

// One threadgroup per row: exp(x - max) / sum, the maximum from -inf and the
// sum from -0, exp in binary64 rounded once.
extern "C" __global__ void __launch_bounds__(1024)
    fk_softmax_f32(const float *__restrict__ x, float *__restrict__ y, fk_softmax_params p) {
  __shared__ float slots[16];
  const uint32_t row = blockIdx.x;
  if (row >= p.rows) return;
  const float *xs = x + (size_t)row * p.n;
  float *ys = y + (size_t)row * p.n;
  const uint32_t packs = p.n / 4;
  float m = -__builtin_inff();
  for (uint32_t j = threadIdx.x; j < packs; j += blockDim.x) {
    float4 v = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)j);
    m = fk::max_number(m, v.x);
    m = fk::max_number(m, v.y);
    m = fk::max_number(m, v.z);
    m = fk::max_number(m, v.w);
  }
  const float top = fk::block_reduce<true>(m, slots);
  float acc = -0.0f;
  for (uint32_t j = threadIdx.x; j < packs; j += blockDim.x) {
    float4 v = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)j);
    acc = acc + fk::exp_once(v.x - top);
    acc = acc + fk::exp_once(v.y - top);
    acc = acc + fk::exp_once(v.z - top);
    acc = acc + fk::exp_once(v.w - top);
  }
  const float total = fk::block_reduce<false>(acc, slots);
  for (uint32_t j = threadIdx.x; j < packs; j += blockDim.x) {
    float4 v = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)j);
    float4 o = make_float4(fk::exp_once(v.x - top) / total, fk::exp_once(v.y - top) / total,
                           fk::exp_once(v.z - top) / total, fk::exp_once(v.w - top) / total);
    *reinterpret_cast<float4 *>(ys + 4 * (size_t)j) = o;
  }
}
