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

#include "../../../include/fkrocm_kernels.h"

#define FK_WAVE 64

// A compile-time choice passed as a value (to a generic lambda).
template <bool B>
struct fk_bool_tag {
  static constexpr bool value = B;
};

namespace fk {

// The greedy token's fold (src/FuryKernel/Program/Eval.hs:681-685: a later
// element wins only if strictly larger) as the maximum of one 64-bit key per
// element: the value's order in the high word (+0 and -0 equal; a NaN at
// index 0 above everything, since nothing is larger than it and it is never
// replaced; a NaN elsewhere below everything, since it never wins), and the
// complement of the index in the low word, so equal values go to the lowest.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
  uint32_t hi;
  if (__builtin_isnan(v)) {
    hi = index == 0 ? 0xFFFFFFFFu : 0u;
  } else {
    const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
    hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - index);
}

// Four 32-bit words in registers: a 16-byte load or store.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));


template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// The sum of a value over the wavefront's 64 lanes, pairwise, neighbours
// first: ((x0 + x1) + (x2 + x3)) + ... (src/FuryKernel/IR.hs:269-283), the same
// value in every lane.  Within each row of 16 lanes by DPP: lane l adds the
// value of lane l ^ 1, then l ^ 2 (quad permutes); after those, the four lanes
// of a quad hold the same bits (IEEE addition commutes), so the half-row
// mirror adds the other quad's sum and the row mirror the other half's.  The
// four rows' sums (lanes 0, 16, 32, 48) are then added as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = v + dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = v + dpp_f<0x141>(v);  // row_half_mirror
  v = v + dpp_f<0x140>(v);  // row_mirror
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// R sums at once, each wave_sum's tree: the DPP steps of the R values
// interleaved so their latencies overlap.
template <int R>
__device__ __forceinline__ void wave_sums(float (&v)[R]) {
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = v[q] + dpp_f<0xB1>(v[q]);
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = v[q] + dpp_f<0x4E>(v[q]);
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = v[q] + dpp_f<0x141>(v[q]);
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = v[q] + dpp_f<0x140>(v[q]);
#pragma unroll
  for (int q = 0; q < R; q++)
    v[q] = (readlane_f(v[q], 0) + readlane_f(v[q], 16)) + (readlane_f(v[q], 32) + readlane_f(v[q], 48));
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

// The wavefront's maximumNumber, every lane, on max_key's integers: within
// rows of 16 lanes by DPP (pairs, quads, halves, rows), then across the four
// rows.  Exact whatever the order.
__device__ __forceinline__ float wave_max(float x) {
  int v = max_key(x);
  v = max(v, dpp_i<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max(v, dpp_i<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max(v, dpp_i<0x141>(v));  // row_half_mirror
  v = max(v, dpp_i<0x140>(v));  // row_mirror
  const int a = __builtin_amdgcn_readlane(v, 0);
  const int b = __builtin_amdgcn_readlane(v, 16);
  const int c = __builtin_amdgcn_readlane(v, 32);
  const int d = __builtin_amdgcn_readlane(v, 48);
  return from_max_key(max(max(a, b), max(c, d)));
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
__device__ __forceinline__ float tanh_once(float x) { return (float)::tanh((double)x); }

// SiLU(a) · b: a / (1 + e^-a), e^-a binary64's rounded once, then times b.
__device__ __forceinline__ float silu_mul(float a, float b) {
  const float e = exp_once(-a);
  const float d = 1.0f + e;
  return (a / d) * b;
}

// GELU in its tanh form (src/FuryKernel/Program/Eval.hs:658-659) in binary32,
// left to right as the formula reads, its constants rounded once and tanh
// binary64's rounded once: (0.5 a) (1 + tanh(c0 (a + ((c1 a) a) a))).
__device__ __forceinline__ float gelu_tanh(float a) {
  const float c0 = 0.7978845608028654f;  // sqrt(2 / pi)
  const float c1 = 0.044715f;
  const float cube = ((c1 * a) * a) * a;
  const float t = tanh_once(c0 * (a + cube));
  return (0.5f * a) * (1.0f + t);
}

// act(a) · b for an activation FK_ACT_*.
__device__ __forceinline__ float act_mul(float a, float b, uint32_t act) {
  return act == FK_ACT_GELU_TANH ? gelu_tanh(a) * b : silu_mul(a, b);
}

// A softcap (Eval.hs:384-390): cap tanh(x / cap).
__device__ __forceinline__ float softcap(float x, float cap) { return cap * tanh_once(x / cap); }

// A bfloat16 element, as its bits (weights of the reference's builder are
// bf16: src/FuryKernel/Program/Build.hs:175-176).
struct bf16_t {
  uint16_t bits;
};

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

// Element j of a head of width d turned by RoPE (NeoX halves, Graph.hs:209-221),
// pair i's cosine and sine from `cs` (the position's row of the RoPE table:
// cos, sin of the binary32 angle position * theta^(-2i/d), each binary64's
// rounded once): (x_j c - x_{j+d/2} s) below the half, (x_j c + x_{j-d/2} s)
// above; pairs past `rotated` stay.
__device__ __forceinline__ float rope_elem(const float *head, uint32_t j, uint32_t d, uint32_t rotated,
                                           const float *__restrict__ cs) {
  const uint32_t half = d / 2;
  const uint32_t i = j < half ? j : j - half;
  if (i >= rotated) return head[j];
  const float c = cs[2 * i];
  const float s = cs[2 * i + 1];
  return j < half ? head[j] * c - head[j + half] * s : head[j] * c + head[j - half] * s;
}

__device__ __forceinline__ uint16_t narrow_cache(float v, bool bf16) { return bf16 ? narrow_bf16(v) : narrow_f16(v); }

__device__ __forceinline__ float widen_cache(uint16_t h, bool bf16) {
  return bf16 ? __uint_as_float((uint32_t)h << 16) : widen_f16(h);
}


}  // namespace fk
