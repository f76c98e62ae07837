// fk_common.h — what every gfx950 kernel of the target shares: the wavefront's
// reductions in the IR's order, the threadgroup reductions of
// src/FuryKernel/Reduce.hs, and the conversions of src/FuryKernel/Numerics.hs.
//
// Arithmetic is Strict (src/FuryKernel/Backend.hs:52-73): the kernels are
// built with -ffp-contract=off and no fast-math, so every float operation
// written is one IEEE 754 operation, rounded once.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FK_WAVE 64

namespace fk {

// Four 32-bit words in registers: a 16-byte load or store.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


// The sum of a value over the wavefront's 64 lanes, in every lane, pairwise,
// neighbours first: ((x0 + x1) + (x2 + x3)) + ... (src/FuryKernel/IR.hs:269-283).
// Step m adds the value of lane l ^ m, which holds the sum of the sibling
// block of m lanes; IEEE addition commutes, so both lanes of a pair hold the
// same bits and every lane ends with the pairwise tree's root.
__device__ __forceinline__ float wave_sum(float v) {
  v = v + __shfl_xor(v, 1);
  v = v + __shfl_xor(v, 2);
  v = v + __shfl_xor(v, 4);
  v = v + __shfl_xor(v, 8);
  v = v + __shfl_xor(v, 16);
  v = v + __shfl_xor(v, 32);
  return v;
}

// IEEE 754-2019 maximumNumber with +0 above -0 (src/FuryKernel/Interp.hs:952-956).
__device__ __forceinline__ float max_number(float x, float y) {
  if (__builtin_isnan(x)) return __builtin_isnan(y) ? __uint_as_float(0x7FC00000u) : y;
  if (__builtin_isnan(y) || x > y) return x;
  if (y > x) return y;
  return __uint_as_float(__float_as_uint(x) & __float_as_uint(y));
}

// maximumNumber as an integer maximum: a float's key orders as the float
// does, -0 below +0, NaN below everything (so a maximum ignores it unless
// every operand is NaN, which gives the quiet NaN back).
__device__ __forceinline__ int max_key(float x) {
  const uint32_t b = __float_as_uint(x);
  return __builtin_isnan(x) ? INT32_MIN : (int)((b & 0x80000000u) ? b ^ 0x7FFFFFFFu : b);
}

__device__ __forceinline__ float from_max_key(int k) {
  if (k == INT32_MIN) return __uint_as_float(0x7FC00000u);
  return __uint_as_float(k < 0 ? (uint32_t)k ^ 0x7FFFFFFFu : (uint32_t)k);
}

// The maximum over the wavefront, pairwise as the sum.
__device__ __forceinline__ float wave_max(float v) {
  v = max_number(v, __shfl_xor(v, 1));
  v = max_number(v, __shfl_xor(v, 2));
  v = max_number(v, __shfl_xor(v, 4));
  v = max_number(v, __shfl_xor(v, 8));
  v = max_number(v, __shfl_xor(v, 16));
  v = max_number(v, __shfl_xor(v, 32));
  return v;
}

// tgReduceSum / tgReduceMax (src/FuryKernel/Reduce.hs:55-85): each wave's
// reduction in its slot; after a barrier the first wave's lane l folds slots
// l, l + 64, ... from the identity (-0 for the sum, -inf for the maximum) and
// reduces once more; every thread gets the result.  `slots` holds one float per
// wave and is reusable when this returns.
template <bool IsMax>
__device__ __forceinline__ float block_reduce(float v, float *slots) {
  const int lane = threadIdx.x & (FK_WAVE - 1);
  const int wave = threadIdx.x / FK_WAVE;
  const int waves = blockDim.x / FK_WAVE;
  float s = IsMax ? wave_max(v) : wave_sum(v);
  if (lane == 0) slots[wave] = s;
  __syncthreads();
  if (wave == 0) {
    float acc = IsMax ? -__builtin_inff() : -0.0f;
    for (int k = lane; k < waves; k += FK_WAVE) acc = IsMax ? max_number(acc, slots[k]) : acc + slots[k];
    float t = IsMax ? wave_max(acc) : wave_sum(acc);
    if (lane == 0) slots[0] = t;
  }
  __syncthreads();
  float total = slots[0];
  __syncthreads();
  return total;
}

// rsqrt, exp: binary64's, rounded once to binary32 (src/FuryKernel/Interp.hs:828-854).
__device__ __forceinline__ float rsqrt_once(float x) { return (float)(1.0 / ::sqrt((double)x)); }
__device__ __forceinline__ float exp_once(float x) { return (float)::exp((double)x); }

// widenF16 (src/FuryKernel/Numerics.hs:51-71): exact; a NaN comes out quiet
// with its sign and payload.
__device__ __forceinline__ float widen_f16(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// narrowF16 (src/FuryKernel/Numerics.hs:100-130): to nearest, ties to even,
// with gradual underflow; a NaN keeps its sign and top payload bits, quiet.
__device__ __forceinline__ uint16_t narrow_f16(float x) {
  uint32_t w = __float_as_uint(x);
  uint32_t sign = (w >> 16) & 0x8000u;
  int e = (int)((w >> 23) & 0xFFu);
  uint32_t m = w & 0x7FFFFFu;
  int unbiased = e - 127;
  uint32_t mag;
  if (e == 0xFF) {
    mag = m ? (0x7E00u | (m >> 13)) : 0x7C00u;
  } else if (unbiased >= 16) {
    mag = 0x7C00u;
  } else if (unbiased >= -14) {
    uint32_t kept = ((uint32_t)(unbiased + 15) << 10) | (m >> 13);
    uint32_t dropped = m & 0x1FFFu;
    mag = kept + ((dropped > 0x1000u || (dropped == 0x1000u && (kept & 1u))) ? 1u : 0u);
  } else {
    int shift = -(unbiased + 1);
    uint32_t full = m | 0x800000u;
    if (shift > 24) {
      mag = 0;
    } else {
      uint32_t kept = full >> shift;
      uint32_t dropped = full & ((1u << shift) - 1u);
      uint32_t half = 1u << (shift - 1);
      mag = kept + ((dropped > half || (dropped == half && (kept & 1u))) ? 1u : 0u);
    }
  }
  return (uint16_t)(sign | mag);
}

// narrowBF16 (src/FuryKernel/Numerics.hs:41-49).
__device__ __forceinline__ uint16_t narrow_bf16(float x) {
  uint32_t w = __float_as_uint(x);
  if (__builtin_isnan(x)) return (uint16_t)((w >> 16) | 0x0040u);
  return (uint16_t)((w + 0x7FFFu + ((w >> 16) & 1u)) >> 16);
}

}  // namespace fk
