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

namespace fk {

// Segments of at most H packs a thread: the thread's packs (t, t + T, ...)
// loaded into registers at once — every load issued before any is used, its
// index clamped into the segment — and both passes made on the registers,
// each in the loop's element order; a pack past the segment is not added
// (a select, so no load sits in a branch) and not stored.
template <int H>
__device__ __forceinline__ void rmsnorm_held(const float *__restrict__ xs, const float *__restrict__ gamma,
                                             float *__restrict__ ys, uint32_t packs, const fk_rmsnorm_params &p,
                                             float *slots) {
  const uint32_t T = blockDim.x, t = threadIdx.x;
  float4 v[H], g[H];
#pragma unroll
  for (int i = 0; i < H; i++) v[i] = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)min(t + i * T, packs - 1));
  if (p.has_gamma) {
#pragma unroll
    for (int i = 0; i < H; i++) g[i] = *reinterpret_cast<const float4 *>(gamma + 4 * (size_t)min(t + i * T, packs - 1));
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < H; i++) {
    float a = acc + v[i].x * v[i].x;
    a = a + v[i].y * v[i].y;
    a = a + v[i].z * v[i].z;
    a = a + v[i].w * v[i].w;
    acc = t + i * T < packs ? a : acc;
  }
  const float total = block_reduce<false>(acc, slots);
  const float scale = rsqrt_once(total / (float)p.seg + p.eps);
#pragma unroll
  for (int i = 0; i < H; i++) {
    if (t + i * T >= packs) break;
    float o[4] = {v[i].x * scale, v[i].y * scale, v[i].z * scale, v[i].w * scale};
    if (p.has_gamma) {
      o[0] = o[0] * g[i].x;
      o[1] = o[1] * g[i].y;
      o[2] = o[2] * g[i].z;
      o[3] = o[3] * g[i].w;
    }
    if (p.factor != 1.0f) {
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = o[e] * p.factor;
    }
    *reinterpret_cast<float4 *>(ys + 4 * (size_t)(t + i * T)) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

}  // namespace fk

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
  const uint32_t held = (packs + blockDim.x - 1) / blockDim.x;  // packs a thread holds
  if (held <= 1) return fk::rmsnorm_held<1>(xs, gamma, ys, packs, p, slots);
  if (held <= 2) return fk::rmsnorm_held<2>(xs, gamma, ys, packs, p, slots);
  if (held <= 4) return fk::rmsnorm_held<4>(xs, gamma, ys, packs, p, slots);
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

// One threadgroup per row: exp(x - max) / sum, the maximum from -inf and the
// sum from -0, exp in binary64 rounded once.
namespace fk {

// Rows of at most H packs a thread, held in registers as RMSNorm's are: the
// maximum, then each element's exp(x - max) once (kept for the output), the
// sum in the loop's order, and the stores of e / sum.
template <int H>
__device__ __forceinline__ void softmax_held(const float *__restrict__ xs, float *__restrict__ ys, uint32_t packs,
                                             float *slots) {
  const uint32_t T = blockDim.x, t = threadIdx.x;
  float4 v[H];
#pragma unroll
  for (int i = 0; i < H; i++) v[i] = *reinterpret_cast<const float4 *>(xs + 4 * (size_t)min(t + i * T, packs - 1));
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < H; i++) {
    float a = max_number(m, v[i].x);
    a = max_number(a, v[i].y);
    a = max_number(a, v[i].z);
    a = max_number(a, v[i].w);
    m = t + i * T < packs ? a : m;
  }
  const float top = block_reduce<true>(m, slots);
  float acc = -0.0f;
  float4 e[H];
#pragma unroll
  for (int i = 0; i < H; i++) {
    e[i] = make_float4(exp_once(v[i].x - top), exp_once(v[i].y - top), exp_once(v[i].z - top),
                       exp_once(v[i].w - top));
    float a = acc + e[i].x;
    a = a + e[i].y;
    a = a + e[i].z;
    a = a + e[i].w;
    acc = t + i * T < packs ? a : acc;
  }
  const float total = block_reduce<false>(acc, slots);
#pragma unroll
  for (int i = 0; i < H; i++) {
    if (t + i * T >= packs) break;
    *reinterpret_cast<float4 *>(ys + 4 * (size_t)(t + i * T)) =
        make_float4(e[i].x / total, e[i].y / total, e[i].z / total, e[i].w / total);
  }
}

}  // namespace fk

extern "C" __global__ void __launch_bounds__(1024)
    fk_softmax_f32(const float *__restrict__ x, float *__restrict__ y, fk_softmax_params p) {
  __shared__ float slots[16];
  const uint32_t row = blockIdx.x;
  if (row >= p.rows) return;
  const float *xs = x + (size_t)row * p.n;
  float *ys = y + (size_t)row * p.n;
  const uint32_t packs = p.n / 4;
  const uint32_t held = (packs + blockDim.x - 1) / blockDim.x;  // packs a thread holds
  if (held <= 1) return fk::softmax_held<1>(xs, ys, packs, slots);
  if (held <= 2) return fk::softmax_held<2>(xs, ys, packs, slots);
  if (held <= 4) return fk::softmax_held<4>(xs, ys, packs, slots);
  if (held <= 8) return fk::softmax_held<8>(xs, ys, packs, slots);
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
