// fk_step.h — one kernel per step shape of a planned decode step
// (src/FuryKernel/Program/Plan.hs:4-55): a step is one launch, its anchors
// set the grid, its recomputed values run in every threadgroup before them,
// its epilogues run on a linear layer's tile.
//
//   fk_step_gemv_*   (fk_step_gemv.h) recompute → anchors → epilogue
//   fk_step_store    recompute RoPE of k → effects: KV stores into ring caches
//   fk_step_attend   recompute RoPE of q → anchor: attention over a split of
//                    positions for one KV head, stored as partials
//   fk_step_combine  attention's combine of its splits
//   fk_step_argmax   the greedy token of a stored row
//   fk_step_act_mul  a stored act·mul, SiLU or GELU-tanh (the light step `store_gelus` plans)
//   fk_step_elementwise, fk_step_gather_*  a light step's Add, ScaleBy,
//                    Standardize, Concat, Gather of stored rows
//   fk_step_advance  the next decode step's token and position, on the device
//
// Arithmetic follows the evaluator's contract (src/FuryKernel/Program/Eval.hs:
// 26-86) in fixed orders, which the oracle restates in C operation for
// operation: GEMV rows in the reference GEMV's order, RMSNorm in tgReduceSum's,
// exp and rsqrt in binary64 rounded once, RoPE's cosines and sines from a
// table of binary64 values rounded once.
#pragma once

#include "fk_common.h"
#include "fk_step_gemv.h"

#define FK_STEP_THREADS 256

// KV stores ----------------------------------------------------------------

// One threadgroup: every element of one row's kv heads, for each store, at
// ((s * kvHeads + h) * length + pos mod length) * headDim (Graph.hs:138-143).
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_store(const float *__restrict__ x0, const float *__restrict__ x1, uint16_t *__restrict__ c0,
                  uint16_t *__restrict__ c1, const uint32_t *__restrict__ position,
                  const uint32_t *__restrict__ slot, const float *__restrict__ rope, fk_step_store_params p) {
  const uint32_t pos = position[0];
  const uint32_t s = slot[0];
  const uint32_t width = p.kv_heads * p.head_dim;
  if (s >= p.slots) return;  // the gate bounds slots: a bad one stores nothing
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  for (uint32_t st = 0; st < p.n_stores; st++) {
    const float *x = st == 0 ? x0 : x1;
    uint16_t *c = st == 0 ? c0 : c1;
    for (uint32_t e = threadIdx.x; e < width; e += blockDim.x) {
      const uint32_t h = e / p.head_dim;
      const uint32_t i = e % p.head_dim;
      const float v = p.rope[st] ? fk::rope_elem(x + h * p.head_dim, i, p.head_dim, p.rotated, cs) : x[e];
      const size_t at = (((size_t)s * p.kv_heads + h) * p.length + pos % p.length) * p.head_dim + i;
      c[at] = fk::narrow_cache(v, p.cache_bf16);
    }
  }
}

// The store into paged pools (Graph.hs:144-152): each element at
// (h * blockSize + pos mod blockSize) * headDim in block table[pos /
// blockSize], the block at pool[b]; nothing stored for a position past the
// table or a block past the pool (the gate bounds both).
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_store_paged(const float *__restrict__ x0, const float *__restrict__ x1,
                        const uint64_t *__restrict__ p0, const uint64_t *__restrict__ p1,
                        const uint32_t *__restrict__ position, const uint32_t *__restrict__ table,
                        const float *__restrict__ rope, fk_step_store_paged_params pp) {
  const fk_step_store_params &p = pp.s;
  const uint32_t pos = position[0];
  const uint32_t bs = pp.g.block_size;
  if (pos / bs >= pp.g.table_len || table[pos / bs] >= pp.g.blocks) return;
  const uint32_t width = p.kv_heads * p.head_dim;
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  const uint32_t b = table[pos / bs];
  for (uint32_t st = 0; st < p.n_stores; st++) {
    const float *x = st == 0 ? x0 : x1;
    uint16_t *c = reinterpret_cast<uint16_t *>((st == 0 ? p0 : p1)[b]);
    for (uint32_t e = threadIdx.x; e < width; e += blockDim.x) {
      const uint32_t h = e / p.head_dim;
      const uint32_t i = e % p.head_dim;
      const float v = p.rope[st] ? fk::rope_elem(x + h * p.head_dim, i, p.head_dim, p.rotated, cs) : x[e];
      c[((size_t)h * bs + pos % bs) * p.head_dim + i] = fk::narrow_cache(v, p.cache_bf16);
    }
  }
}

// Attention: the split attention and the combine (fk_attention.h) -----------

#include "fk_attention.h"

extern "C" __global__ void __launch_bounds__(FK_ATTN_THREADS)
    fk_step_attend(const float *__restrict__ q, const float *__restrict__ knew, const float *__restrict__ vnew,
                   uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                   const uint32_t *__restrict__ slot, const float *__restrict__ rope, float *__restrict__ partials,
                   const uint32_t *__restrict__ reach, fk_step_attend_params p) {
  fk::step_attend(q, knew, vnew, kc, vc, position, slot, rope, partials, reach, p);
}

// The attention in wide splits (fk_attention.h): 32 positions a wavefront,
// up to 16 wavefronts a threadgroup, the LDS fk::wide_lds_floats(waves) floats.
extern "C" __global__ void __launch_bounds__(FK_WAVE * FK_WIDE_MAX_WAVES)
    fk_step_attend_wide(const float *__restrict__ q, const float *__restrict__ knew, const float *__restrict__ vnew,
                        uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                        const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                        float *__restrict__ partials, const uint32_t *__restrict__ reach,
                        fk_step_attend_params p) {
  fk::step_attend_wide(q, knew, vnew, kc, vc, position, slot, rope, partials, reach, p);
}

extern "C" __global__ void __launch_bounds__(FK_ATTN_THREADS)
    fk_step_attend_paged(const float *__restrict__ q, const float *__restrict__ knew,
                         const float *__restrict__ vnew, const uint64_t *__restrict__ kpool,
                         const uint64_t *__restrict__ vpool, const uint32_t *__restrict__ position,
                         const uint32_t *__restrict__ table, const float *__restrict__ rope,
                         float *__restrict__ partials, const uint32_t *__restrict__ reach,
                         fk_step_attend_paged_params p) {
  fk::step_attend_paged(q, knew, vnew, kpool, vpool, position, table, rope, partials, reach, p);
}

extern "C" __global__ void __launch_bounds__(FK_WAVE)
    fk_step_combine(const float *__restrict__ partials, float *__restrict__ out, fk_step_combine_params p) {
  fk::step_combine(partials, out, p);
}

namespace fk {
// Of two (value, index) candidates, the larger value; of equal values (or
// values neither larger), the lower index: the fold of Eval.hs:681-685 where
// a later element wins only if strictly larger.
__device__ __forceinline__ void argmax_merge(float &v, uint32_t &i, float ov, uint32_t oi) {
  if (oi == 0xFFFFFFFFu) return;
  if (i == 0xFFFFFFFFu) {
    v = ov;
    i = oi;
    return;
  }
  const bool take = oi < i ? !(v > ov) : ov > v;
  if (take) {
    v = ov;
    i = oi;
  }
}
}  // namespace fk

extern "C" __global__ void __launch_bounds__(1024)
    fk_step_argmax(const float *__restrict__ x, uint32_t *__restrict__ out, fk_step_argmax_params p) {
  __shared__ float bv[16];
  __shared__ uint32_t bi[16];
  float v = -__builtin_inff();
  uint32_t idx = 0xFFFFFFFFu;
  for (uint32_t i = threadIdx.x; i < p.n; i += blockDim.x) fk::argmax_merge(v, idx, x[i], i);
  for (int m = 1; m < FK_WAVE; m <<= 1) {
    const float ov = __shfl_xor(v, m);
    const uint32_t oi = __shfl_xor(idx, m);
    fk::argmax_merge(v, idx, ov, oi);
  }
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t wave = threadIdx.x / FK_WAVE;
  if (lane == 0) {
    bv[wave] = v;
    bi[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float fv = bv[0];
    uint32_t fi = bi[0];
    for (uint32_t w2 = 1; w2 < blockDim.x / FK_WAVE; w2++) fk::argmax_merge(fv, fi, bv[w2], bi[w2]);
    out[0] = fi;
  }
}

extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_act_mul(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ y,
                    fk_step_act_mul_params p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  if (p.half) {
    const size_t at = (size_t)(i / p.half) * 2 * p.half + i % p.half;
    y[i] = fk::act_mul(a[at], a[at + p.half], p.act);
  } else {
    y[i] = fk::act_mul(a[i], b[p.b_off + i], p.act);
  }
}

// Routing: one wavefront, k rounds of the wavefront's largest key among the
// logits not yet taken (the argmax keys, a NaN's the lowest), then lane 0's
// weights.
extern "C" __global__ void __launch_bounds__(FK_WAVE)
    fk_step_route(const float *__restrict__ x, const float *__restrict__ scale, uint32_t *__restrict__ ids,
                  float *__restrict__ ws, fk_step_route_params p) {
  const uint32_t lane = threadIdx.x;
  uint32_t taken[8];
  float tv[8];
#pragma unroll
  for (int r = 0; r < 8; r++) taken[r] = 0xFFFFFFFFu, tv[r] = 0.0f;
#pragma unroll
  for (int r = 0; r < 8; r++) {
    if ((uint32_t)r < p.k) {
      uint64_t best = 0;
      for (uint32_t i = lane; i < p.n; i += FK_WAVE) {
        bool seen = false;
#pragma unroll
        for (int q = 0; q < 8; q++) seen |= q < r && taken[q] == i;
        const float v = x[i];
        const uint64_t key = __builtin_isnan(v) ? (uint64_t)(0xFFFFFFFFu - i) : fk::argmax_key(v, i);
        if (!seen && key > best) best = key;
      }
#pragma unroll
      for (int m = 1; m < FK_WAVE; m <<= 1) {
        const uint64_t o = __shfl_xor(best, m);
        best = o > best ? o : best;
      }
      taken[r] = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu);
      tv[r] = x[taken[r]];
    }
  }
  if (lane == 0) {
    float e[8], total = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; r++) {
      if ((uint32_t)r < p.k) {
        e[r] = fk::exp_once(tv[r] - tv[0]);
        total = total + e[r];
      }
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      if ((uint32_t)r < p.k) {
        float w = e[r] / total;
        if (p.has_scale) w = w * scale[taken[r]];
        ids[r] = taken[r];
        ws[r] = w;
      }
    }
  }
}

// CombineRanks, and the residual add after it.
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_combine_ranks(const float *__restrict__ w, const float *__restrict__ x, const float *__restrict__ res,
                          float *__restrict__ y, fk_step_combine_ranks_params p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.seg) return;
  float acc = w[0] * x[i];
  for (uint32_t r = 1; r < p.ranks; r++) acc = acc + w[r] * x[(size_t)r * p.seg + i];
  if (p.residual) acc = res[i] + acc;
  y[i] = acc;
}

// A light step's elementwise value of stored rows (Add, ScaleBy,
// Standardize, Concat); binary32 operations in the evaluator's order.
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_elementwise(const float *__restrict__ a, const float *__restrict__ b, const float *__restrict__ c,
                        float *__restrict__ y, fk_step_elementwise_params p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  switch (p.op) {
    case FK_ELT_ADD: y[i] = a[i] + b[i]; break;
    case FK_ELT_SCALE: y[i] = a[i] * b[0]; break;
    case FK_ELT_STANDARDIZE: {
      const uint32_t j = i % p.width;
      y[i] = (p.factor * a[i] - b[j]) * c[j];
      break;
    }
    default: {  // FK_ELT_CONCAT
      const uint32_t w = p.width + p.width_b;
      const uint32_t r = i / w, j = i % w;
      y[i] = j < p.width ? a[(size_t)r * p.width + j] : b[(size_t)r * p.width_b + (j - p.width)];
    }
  }
}

// Gather: each row's tokens' table rows summed from +0 in order, then
// scaled.
template <typename WT>
__device__ __forceinline__ void step_gather(const WT *__restrict__ table, const uint32_t *__restrict__ tokens,
                                            float *__restrict__ y, const fk_step_gather_params &p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.rows * p.width) return;
  const uint32_t r = i / p.width, j = i % p.width;
  float s = 0.0f;
  for (uint32_t t = 0; t < p.count; t++) {
    const uint32_t tok = min(tokens[(size_t)r * p.count + t], p.table_rows - 1);
    s = s + fk::to_float(table[(size_t)tok * p.width + j]);
  }
  y[i] = s * p.factor;
}

#define FK_STEP_GATHER(NAME, WT)                                                                            \
  extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)                                           \
      NAME(const WT *__restrict__ table, const uint32_t *__restrict__ tokens, float *__restrict__ y,      \
           fk_step_gather_params p) {                                                                      \
    step_gather<WT>(table, tokens, y, p);                                                                  \
  }
FK_STEP_GATHER(fk_step_gather_f32, float)
FK_STEP_GATHER(fk_step_gather_f16, _Float16)
FK_STEP_GATHER(fk_step_gather_bf16, fk::bf16_t)

// The next decode step's inputs: its token is this step's greedy token, its
// position `step` more.
extern "C" __global__ void fk_step_advance(const uint32_t *__restrict__ next_token, uint32_t *__restrict__ token,
                                           uint32_t *__restrict__ position, fk_step_advance_params p) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    token[0] = next_token[0];
    position[0] = (position[0] + p.step) % p.context;
  }
}

// Synthetic weights: element i is std * N(0, 1), the normal by Box-Muller from
// the SplitMix64 stream of `seed` (uniforms (u >> 40) 2^-24), rounded once to
// the element type.
extern "C" __global__ void __launch_bounds__(256) fk_init_normal(void *__restrict__ dst, fk_init_normal_params p) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < p.count;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t pair = i / 2;
    auto mix = [](uint64_t z) {
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      return z ^ (z >> 31);
    };
    const uint64_t golden = 0x9E3779B97F4A7C15ull;
    const double u1 = (double)(mix(p.seed + (2 * pair + 1) * golden) >> 40) * 0x1p-24;
    const double u2 = (double)(mix(p.seed + (2 * pair + 2) * golden) >> 40) * 0x1p-24;
    const double r = ::sqrt(-2.0 * ::log(1.0 - u1));
    const double t = 6.283185307179586 * u2;
    const double z = (i & 1) ? r * ::sin(t) : r * ::cos(t);
    const float v = (float)(z * (double)p.std);
    if (p.dtype == 1)
      reinterpret_cast<uint16_t *>(dst)[i] = fk::narrow_f16(v);
    else if (p.dtype == 2)
      reinterpret_cast<uint16_t *>(dst)[i] = fk::narrow_bf16(v);
    else
      reinterpret_cast<float *>(dst)[i] = v;
  }
}
