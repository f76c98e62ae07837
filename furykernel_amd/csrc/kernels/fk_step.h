// fk_step.h — one kernel per step shape of a planned decode step
// (src/FuryKernel/Program/Plan.hs:4-55): a step is one launch, its anchors
// set the grid, its recomputed values run in every threadgroup before them,
// its epilogues run on a linear layer's tile.
//
//   fk_step_gemv_*   recompute (RMSNorm of a stored row or a gathered
//                    embedding row, SiLU·mul of two stored rows) → anchors
//                    (linear layers sharing the input) → epilogue (residual add)
//   fk_step_store    recompute RoPE of k → effects: KV stores into ring caches
//   fk_step_attend   recompute RoPE of q → anchor: attention over a split of
//                    positions for one KV head, stored as partials
//   fk_step_combine  attention's combine of its splits
//   fk_step_argmax   the greedy token of a stored row
//   fk_step_silu_mul a stored SiLU·mul (the light step `store_gelus` plans)
//   fk_step_advance  the next decode step's token and position, on the device
//
// Arithmetic follows the evaluator's contract (src/FuryKernel/Program/Eval.hs:
// 26-86) in fixed orders, which the oracle restates in C operation for
// operation: GEMV rows in the reference GEMV's order, RMSNorm in tgReduceSum's,
// exp/sin/cos/pow in binary64 rounded once.
#pragma once

#include "fk_common.h"
#include "fk_gemv.h"

#define FK_STEP_MAX_K 8192
#define FK_STEP_THREADS 256

// Prologue modes: how a GEMV step's threadgroups make the anchors' input row.
enum : uint32_t {
  FK_PRO_STORED = 0,          // x = src
  FK_PRO_RMSNORM = 1,         // x = rmsnorm(src) * gamma * factor
  FK_PRO_GATHER = 2,          // x = table[token] * gfactor
  FK_PRO_GATHER_RMSNORM = 3,  // x = rmsnorm(table[token] * gfactor) * gamma * factor
  FK_PRO_SILU_MUL = 4,        // x = silu(src) * src2
};

// Epilogue modes: elementwise work on the anchor's tile.
enum : uint32_t {
  FK_EPI_NONE = 0,
  FK_EPI_ADD_STORED = 1,  // out = res + tile
  FK_EPI_ADD_GATHER = 2,  // out = table[token] * gfactor + tile
};

struct fk_step_gemv_params {
  uint32_t n_anchors;  // 1 to 3
  uint32_t rows[3];    // each anchor's outputs
  uint32_t first_group[4];  // anchor j's threadgroups are [first_group[j], first_group[j+1])
  uint32_t k;          // the input row's width
  uint32_t pro_mode;
  uint32_t seg;        // RMSNorm's segment (k, one segment)
  float eps;
  float factor;        // RMSNorm's factor
  float gfactor;       // the gather's factor
  uint32_t has_gamma;
  uint32_t epi_mode;
  uint32_t store_tile;  // the anchors' own values are stored (into y[j])
  uint32_t table_rows;  // the gathered table's rows: a token past them reads its last (the engine refuses one)
};

namespace fk {

// The row of `table` a token names, times the factor: a gather of one row
// (src/FuryKernel/Program/Eval.hs:528-535).
template <typename TT>
__device__ __forceinline__ float gathered(const TT *__restrict__ table, uint32_t token, uint32_t k, uint32_t i,
                                          float f) {
  return (float)table[(size_t)token * k + i] * f;
}

// RMSNorm of a row held in LDS `xs` (k elements, segments of `seg`), in place:
// per segment the threads' sums of squares over packs of 4 in tgReduceSum's
// order, scale = rsqrt(sum / seg + eps) in binary64 rounded once, then
// ((x * scale) * gamma) * factor.
__device__ __forceinline__ void rmsnorm_lds(float *xs, uint32_t k, uint32_t seg, float eps, float factor,
                                            const float *__restrict__ gamma, float *slots) {
  for (uint32_t s0 = 0; s0 < k; s0 += seg) {
    const uint32_t packs = seg / 4;
    float acc = 0.0f;
    for (uint32_t j = threadIdx.x; j < packs; j += blockDim.x) {
      const float *v = xs + s0 + 4 * j;
      acc = acc + v[0] * v[0];
      acc = acc + v[1] * v[1];
      acc = acc + v[2] * v[2];
      acc = acc + v[3] * v[3];
    }
    const float total = block_reduce<false>(acc, slots);
    const float scale = rsqrt_once(total / (float)seg + eps);
    for (uint32_t i = threadIdx.x; i < seg; i += blockDim.x) {
      float v = xs[s0 + i] * scale;
      if (gamma) v = v * gamma[i];
      if (factor != 1.0f) v = v * factor;
      xs[s0 + i] = v;
    }
    __syncthreads();
  }
}

// SiLU(a) · b: a / (1 + e^-a), e^-a binary64's rounded once, then times b.
__device__ __forceinline__ float silu_mul(float a, float b) {
  const float e = exp_once(-a);
  const float d = 1.0f + e;
  return (a / d) * b;
}

}  // namespace fk

// One wavefront's rows of a GEMV step: R rows of one anchor, x in LDS.  The
// first PF packs of every row are loaded before the prologue runs (weights
// don't depend on it), so the prologue hides their latency.
template <typename WT, int P, int R, int PF>
__device__ __forceinline__ void step_gemv_body(const WT *const *__restrict__ ws, float *const *__restrict__ ys,
                                               const float *__restrict__ src, const float *__restrict__ src2,
                                               const float *__restrict__ gamma, const WT *__restrict__ table,
                                               const uint32_t *__restrict__ token, const float *__restrict__ res,
                                               const WT *__restrict__ res_table, const uint32_t *__restrict__ res_token,
                                               float *__restrict__ epi_out, const fk_step_gemv_params &p) {
  __shared__ float xs[FK_STEP_MAX_K];
  __shared__ float slots[16];
  constexpr int C = P / 4;
  // Which anchor and rows this threadgroup takes.
  uint32_t a = 0;
  while (a + 1 < p.n_anchors && blockIdx.x >= p.first_group[a + 1]) a++;
  const uint32_t n = p.rows[a];
  const uint32_t k = p.k;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t wave = threadIdx.x / FK_WAVE;
  const uint32_t waves = blockDim.x / FK_WAVE;
  const uint32_t row0 = ((blockIdx.x - p.first_group[a]) * waves + wave) * R;
  const bool active = row0 < n;
  const WT *w = ws[a];
  const uint32_t packs = k / P;
  const WT *wr[R];
#pragma unroll
  for (int q = 0; q < R; q++) wr[q] = w + (size_t)min(row0 + q, n - 1) * k;

  // Prefetch: the first PF packs of each row, as 16-byte words.
  constexpr int U = P * sizeof(WT) / 16;
  uint4 pre[PF][R][U];
#pragma unroll
  for (int it = 0; it < PF; it++) {
    const uint32_t j = lane + it * FK_WAVE;
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
      for (int u = 0; u < U; u++)
        pre[it][q][u] = (active && j < packs) ? reinterpret_cast<const uint4 *>(wr[q] + (size_t)j * P)[u]
                                              : make_uint4(0, 0, 0, 0);
  }

  // Prologue: the anchors' input row, into LDS.
  const uint32_t tok =
      (p.pro_mode == FK_PRO_GATHER || p.pro_mode == FK_PRO_GATHER_RMSNORM) ? min(token[0], p.table_rows - 1) : 0;
  for (uint32_t i = threadIdx.x; i < k; i += blockDim.x) {
    float v;
    switch (p.pro_mode) {
      case FK_PRO_GATHER:
      case FK_PRO_GATHER_RMSNORM: v = fk::gathered(table, tok, k, i, p.gfactor); break;
      case FK_PRO_SILU_MUL: v = fk::silu_mul(src[i], src2[i]); break;
      default: v = src[i]; break;
    }
    xs[i] = v;
  }
  __syncthreads();
  if (p.pro_mode == FK_PRO_RMSNORM || p.pro_mode == FK_PRO_GATHER_RMSNORM)
    fk::rmsnorm_lds(xs, k, p.seg, p.eps, p.factor, p.has_gamma ? gamma : nullptr, slots);
  if (!active) return;

  // The rows, in the reference GEMV's order.
  float acc[R][C];
#pragma unroll
  for (int q = 0; q < R; q++)
#pragma unroll
    for (int c = 0; c < C; c++) acc[q][c] = 0.0f;
  auto consume = [&](uint32_t j, const uint4 (&wv4)[R][U]) {
    float xv[P];
#pragma unroll
    for (int e = 0; e < P; e++) xv[e] = xs[j * P + e];
#pragma unroll
    for (int q = 0; q < R; q++) {
      float wv[P];
      fk::unpack<P>(wv4[q], wv, WT{});
#pragma unroll
      for (int c = 0; c < C; c++) {
        float p0 = xv[4 * c] * wv[4 * c];
        float p1 = xv[4 * c + 1] * wv[4 * c + 1];
        float p2 = xv[4 * c + 2] * wv[4 * c + 2];
        float p3 = xv[4 * c + 3] * wv[4 * c + 3];
        acc[q][c] = acc[q][c] + ((p0 + p1) + (p2 + p3));
      }
    }
  };
#pragma unroll
  for (int it = 0; it < PF; it++) {
    const uint32_t j = lane + it * FK_WAVE;
    if (j < packs) consume(j, pre[it]);
  }
#pragma unroll 4
  for (uint32_t j = lane + PF * FK_WAVE; j < packs; j += FK_WAVE) {
    uint4 wv4[R][U];
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
      for (int u = 0; u < U; u++)
        wv4[q][u] = reinterpret_cast<const uint4 *>(wr[q] + (size_t)j * P)[u];
    consume(j, wv4);
  }

  const uint32_t rtok = (p.epi_mode == FK_EPI_ADD_GATHER) ? min(res_token[0], p.table_rows - 1) : 0;
#pragma unroll
  for (int q = 0; q < R; q++) {
    float t = acc[q][0];
#pragma unroll
    for (int c = 1; c < C; c++) t = t + acc[q][c];
    t = fk::wave_sum(t);
    const uint32_t row = row0 + q;
    if (lane == 0 && row < n) {
      if (p.store_tile) ys[a][row] = t;
      if (p.epi_mode == FK_EPI_ADD_STORED) {
        epi_out[row] = res[row] + t;
      } else if (p.epi_mode == FK_EPI_ADD_GATHER) {
        epi_out[row] = fk::gathered(res_table, rtok, n, row, p.gfactor) + t;
      }
    }
  }
}

// Buffers in binding order, then the parameter struct.
#define FK_STEP_GEMV_ENTRY(NAME, WT, P, R, PF)                                                                      \
  extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)                                                     \
      NAME(const WT *__restrict__ w0, const WT *__restrict__ w1, const WT *__restrict__ w2, float *__restrict__ y0, \
           float *__restrict__ y1, float *__restrict__ y2, const float *__restrict__ src,                          \
           const float *__restrict__ src2, const float *__restrict__ gamma, const WT *__restrict__ table,           \
           const uint32_t *__restrict__ token, const float *__restrict__ res, const WT *__restrict__ res_table,     \
           const uint32_t *__restrict__ res_token, float *__restrict__ epi_out, fk_step_gemv_params p) {           \
    const WT *ws[3] = {w0, w1, w2};                                                                                 \
    float *ys[3] = {y0, y1, y2};                                                                                    \
    step_gemv_body<WT, P, R, PF>(ws, ys, src, src2, gamma, table, token, res, res_table, res_token, epi_out, p);   \
  }

FK_STEP_GEMV_ENTRY(fk_step_gemv_f16_r1, _Float16, 8, 1, 4)
FK_STEP_GEMV_ENTRY(fk_step_gemv_f16_r2, _Float16, 8, 2, 4)
FK_STEP_GEMV_ENTRY(fk_step_gemv_f32_r1, float, 4, 1, 4)

// KV stores ----------------------------------------------------------------

struct fk_step_store_params {
  uint32_t n_stores;    // 1 or 2
  uint32_t rope[2];     // store j's value is RoPE'd first (its source is k)
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t length;      // the ring's positions
  uint32_t slots;       // the ring's sequences
  uint32_t rotated;     // pairs turned
  float theta;
  uint32_t cache_bf16;  // the caches round to bf16 (else f16)
};

namespace fk {

// The frequency of pair i of a head of width d: theta^(-2i/d) in binary64,
// rounded once.
__device__ __forceinline__ float rope_freq(float theta, uint32_t i, uint32_t d) {
  return (float)::pow((double)theta, -(double)(2 * i) / (double)d);
}

// Element j of a head turned by `position` (NeoX halves, Graph.hs:209-221):
// angle = position * freq in binary32, its cosine and sine binary64's rounded
// once; (x_j c - x_{j+d/2} s) below the half, (x_j c + x_{j-d/2} s) above.
__device__ __forceinline__ float rope_elem(const float *head, uint32_t j, uint32_t d, uint32_t rotated,
                                           uint32_t position, float theta) {
  const uint32_t half = d / 2;
  const uint32_t i = j < half ? j : j - half;
  if (i >= rotated) return head[j];
  const float angle = (float)position * rope_freq(theta, i, d);
  const float c = (float)::cos((double)angle);
  const float s = (float)::sin((double)angle);
  return j < half ? head[j] * c - head[j + half] * s : head[j] * c + head[j - half] * s;
}

__device__ __forceinline__ uint16_t narrow_cache(float v, bool bf16) { return bf16 ? narrow_bf16(v) : narrow_f16(v); }

}  // namespace fk

// One threadgroup: every element of one row's kv heads, for each store.
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_store(const float *__restrict__ x0, const float *__restrict__ x1, uint16_t *__restrict__ c0,
                  uint16_t *__restrict__ c1, const uint32_t *__restrict__ position,
                  const uint32_t *__restrict__ slot, fk_step_store_params p) {
  const uint32_t pos = position[0];
  const uint32_t s = slot[0];
  const uint32_t width = p.kv_heads * p.head_dim;
  if (s >= p.slots) return;  // the gate bounds slots; a bad one stores nothing
  for (uint32_t st = 0; st < p.n_stores; st++) {
    const float *x = st == 0 ? x0 : x1;
    uint16_t *c = st == 0 ? c0 : c1;
    for (uint32_t e = threadIdx.x; e < width; e += blockDim.x) {
      const uint32_t h = e / p.head_dim;
      const uint32_t i = e % p.head_dim;
      const float v = p.rope[st] ? fk::rope_elem(x + h * p.head_dim, i, p.head_dim, p.rotated, pos, p.theta) : x[e];
      // Ring: ((s * kvHeads + h) * length + pos mod length) * headDim (Graph.hs:138-143).
      const size_t at = (((size_t)s * p.kv_heads + h) * p.length + pos % p.length) * p.head_dim + i;
      c[at] = fk::narrow_cache(v, p.cache_bf16);
    }
  }
}

// Attention ----------------------------------------------------------------

#define FK_ATTN_SPLIT 128
#define FK_ATTN_MAX_GROUP 8
#define FK_ATTN_MAX_DIM 64

struct fk_step_attend_params {
  uint32_t heads;
  uint32_t kv_heads;
  uint32_t head_dim;  // at most 64
  uint32_t length;    // the ring's positions
  uint32_t slots;
  uint32_t splits;    // threadgroups per kv head; split t covers positions [128 t, 128 t + 128)
  uint32_t rope;      // q is RoPE'd first
  uint32_t rotated;
  float theta;
  float scale;        // the attention's scale, rounded once to binary32
  uint32_t window;    // 0: none
  uint32_t cache_bf16;
};

namespace fk {
__device__ __forceinline__ float widen_cache(uint16_t h, bool bf16) {
  return bf16 ? __uint_as_float((uint32_t)h << 16) : widen_f16(h);
}
}  // namespace fk

// Threadgroup (kv head g, split t): the scores of the group's query heads over
// the split's positions, each head's maximum over the split, the weights
// exp(score - max), their sum and the weighted sum of the values, stored as
// partials: per (head, split) [max, sum, acc[head_dim]].
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_attend(const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
                   const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot,
                   float *__restrict__ partials, fk_step_attend_params p) {
  constexpr uint32_t KS = FK_ATTN_MAX_DIM + 2;  // a key row's stride in LDS, past the banks' period
  __shared__ float qs[FK_ATTN_MAX_GROUP * FK_ATTN_MAX_DIM];
  __shared__ uint16_t ks[FK_ATTN_SPLIT * KS];
  __shared__ uint16_t vs[FK_ATTN_SPLIT * FK_ATTN_MAX_DIM];
  __shared__ float wt[FK_ATTN_MAX_GROUP * FK_ATTN_SPLIT];
  __shared__ float mx[FK_ATTN_MAX_GROUP];
  const uint32_t g = blockIdx.x / p.splits;
  const uint32_t t = blockIdx.x % p.splits;
  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t d = p.head_dim;
  const uint32_t pos = position[0];
  const uint32_t s = slot[0] < p.slots ? slot[0] : 0;
  const bool bf16 = p.cache_bf16 != 0;
  // Positions [first, pos], this split's part of them.
  const uint32_t first = (p.window && pos + 1 > p.window) ? pos + 1 - p.window : 0;
  const uint32_t lo = max(first, t * FK_ATTN_SPLIT);
  const uint32_t hi = min(pos + 1, (t + 1) * FK_ATTN_SPLIT);
  const uint32_t count = hi > lo ? hi - lo : 0;
  for (uint32_t e = threadIdx.x; e < group * d; e += blockDim.x) {
    const float *head = q + (size_t)(g * group + e / d) * d;
    qs[e] = p.rope ? fk::rope_elem(head, e % d, d, p.rotated, pos, p.theta) : head[e % d];
  }
  const size_t base = ((size_t)s * p.kv_heads + g) * p.length;
  for (uint32_t e = threadIdx.x; e < count * d; e += blockDim.x) {
    const uint32_t r = e / d;
    const size_t at = (base + (lo + r) % p.length) * d + e % d;
    ks[r * KS + e % d] = kc[at];
    vs[e] = vc[at];
  }
  __syncthreads();
  // Scores: (sum over i in order of q_i k_i) * scale.
  for (uint32_t e = threadIdx.x; e < group * count; e += blockDim.x) {
    const uint32_t h = e / count;
    const uint32_t r = e % count;
    float dot = 0.0f;
    for (uint32_t i = 0; i < d; i++) dot = dot + qs[h * d + i] * fk::widen_cache(ks[r * KS + i], bf16);
    wt[h * FK_ATTN_SPLIT + r] = dot * p.scale;
  }
  __syncthreads();
  if (threadIdx.x < group) {
    float m = -__builtin_inff();
    for (uint32_t r = 0; r < count; r++) m = fk::max_number(m, wt[threadIdx.x * FK_ATTN_SPLIT + r]);
    mx[threadIdx.x] = m;
  }
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < group * count; e += blockDim.x) {
    const uint32_t h = e / count;
    const uint32_t r = e % count;
    wt[h * FK_ATTN_SPLIT + r] = fk::exp_once(wt[h * FK_ATTN_SPLIT + r] - mx[h]);
  }
  __syncthreads();
  // Thread (h, i): the weights' sum and the weighted values, in order of position.
  for (uint32_t e = threadIdx.x; e < group * d; e += blockDim.x) {
    const uint32_t h = e / d;
    const uint32_t i = e % d;
    float l = 0.0f;
    float acc = 0.0f;
    for (uint32_t r = 0; r < count; r++) {
      const float w = wt[h * FK_ATTN_SPLIT + r];
      l = l + w;
      acc = acc + w * fk::widen_cache(vs[r * d + i], bf16);
    }
    float *out = partials + ((size_t)(g * group + h) * p.splits + t) * (d + 2);
    if (i == 0) {
      out[0] = mx[h];
      out[1] = l;
    }
    out[2 + i] = acc;
  }
}

struct fk_step_combine_params {
  uint32_t heads;
  uint32_t head_dim;
  uint32_t splits;
};

// Thread (h, i): the splits combined once, in split order: M the largest
// maximum, w_t = exp(max_t - M), out = (sum_t acc_t w_t) / (sum_t l_t w_t).
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_combine(const float *__restrict__ partials, float *__restrict__ out, fk_step_combine_params p) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= p.heads * p.head_dim) return;
  const uint32_t h = e / p.head_dim;
  const uint32_t i = e % p.head_dim;
  const uint32_t stride = p.head_dim + 2;
  const float *ph = partials + (size_t)h * p.splits * stride;
  float m = -__builtin_inff();
  for (uint32_t t = 0; t < p.splits; t++) m = fk::max_number(m, ph[t * stride]);
  float l = 0.0f;
  float acc = 0.0f;
  for (uint32_t t = 0; t < p.splits; t++) {
    const float w = fk::exp_once(ph[t * stride] - m);
    l = l + ph[t * stride + 1] * w;
    acc = acc + ph[t * stride + 2 + i] * w;
  }
  out[e] = acc / l;
}

// Greedy token ------------------------------------------------------------

struct fk_step_argmax_params {
  uint32_t n;
};

// The index of the row's largest element, ties to the lowest
// (src/FuryKernel/Program/Eval.hs:681-685): thread t scans t, t + T, ...; then
// pairs combine, the later winning only if strictly larger.
extern "C" __global__ void __launch_bounds__(1024)
    fk_step_argmax(const float *__restrict__ x, uint32_t *__restrict__ out, fk_step_argmax_params p) {
  __shared__ float bv[1024];
  __shared__ uint32_t bi[1024];
  float v = -__builtin_inff();
  uint32_t idx = 0xFFFFFFFFu;
  for (uint32_t i = threadIdx.x; i < p.n; i += blockDim.x) {
    const float c = x[i];
    if (idx == 0xFFFFFFFFu || c > v) {
      v = c;
      idx = i;
    }
  }
  bv[threadIdx.x] = v;
  bi[threadIdx.x] = idx;
  __syncthreads();
  for (uint32_t w = blockDim.x / 2; w > 0; w /= 2) {
    if (threadIdx.x < w) {
      const float ov = bv[threadIdx.x + w];
      const uint32_t oi = bi[threadIdx.x + w];
      const uint32_t mi = bi[threadIdx.x];
      // The element of the lower index wins unless the other is strictly larger.
      const bool other_lower = oi < mi;
      const bool take = oi != 0xFFFFFFFFu &&
                        (mi == 0xFFFFFFFFu || (other_lower ? !(bv[threadIdx.x] > ov) : ov > bv[threadIdx.x]));
      if (take) {
        bv[threadIdx.x] = ov;
        bi[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = bi[0];
}

struct fk_step_silu_mul_params {
  uint32_t n;
};

extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_silu_mul(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ y,
                     fk_step_silu_mul_params p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < p.n) y[i] = fk::silu_mul(a[i], b[i]);
}

struct fk_step_advance_params {
  uint32_t context;  // positions wrap below this
  uint32_t step;     // positions advance by this (0 holds the position)
};

// The next decode step's inputs: its token is this step's greedy token, its
// position `step` more.
extern "C" __global__ void fk_step_advance(const uint32_t *__restrict__ next_token, uint32_t *__restrict__ token,
                                           uint32_t *__restrict__ position, fk_step_advance_params p) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    token[0] = next_token[0];
    position[0] = (position[0] + p.step) % p.context;
  }
}

struct fk_init_normal_params {
  uint64_t count;
  uint64_t seed;
  float std;
  uint32_t f16;  // store binary16 (else binary32)
};

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
    if (p.f16)
      reinterpret_cast<uint16_t *>(dst)[i] = fk::narrow_f16(v);
    else
      reinterpret_cast<float *>(dst)[i] = v;
  }
}
