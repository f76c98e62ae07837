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
// exp and rsqrt in binary64 rounded once, RoPE's cosines and sines from a
// table of binary64 values rounded once.
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
  uint32_t first_group[4];  // anchor j's row blocks are [first_group[j], first_group[j+1])
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

// An anchor's pointer or count by index, without indexing an array: a
// dynamically indexed array of kernel pointers would lose their address space
// (its loads would become flat loads, which wait with LDS traffic).
template <typename T>
__device__ __forceinline__ T pick3(uint32_t a, T x0, T x1, T x2) {
  return a == 0 ? x0 : (a == 1 ? x1 : x2);
}

// Which anchor row r of the numbered rows belongs to.
__device__ __forceinline__ uint32_t anchor_of(uint32_t r, const fk_step_gemv_params &p) {
  return (p.n_anchors > 1 && r >= p.first_group[1] ? 1u : 0u) + (p.n_anchors > 2 && r >= p.first_group[2] ? 1u : 0u);
}

}  // namespace fk

// The prologue of a GEMV step in two halves, so that its loads are issued
// before the weights' and its arithmetic runs while the weights stream in
// (the wave waits for loads in the order it issued them).  Thread t holds
// packs t, t + T, ... of the row (NPK of them at most, 4 elements each), the
// order RMSNorm's sum of squares takes them in.
template <typename WT, int NPK>
struct Prologue {
  float4 x[NPK];
  float4 x2[NPK];
  float4 g[NPK];

  __device__ __forceinline__ void load(const float *__restrict__ src, const float *__restrict__ src2,
                                       const float *__restrict__ gamma, const WT *__restrict__ table,
                                       const uint32_t *__restrict__ token, const fk_step_gemv_params &p) {
    const uint32_t packs = p.k / 4;
    const bool gather = p.pro_mode == FK_PRO_GATHER || p.pro_mode == FK_PRO_GATHER_RMSNORM;
    const uint32_t tok = gather ? min(token[0], p.table_rows - 1) : 0;
#pragma unroll
    for (int m = 0; m < NPK; m++) {
      const uint32_t j = threadIdx.x + m * blockDim.x;
      const bool in = j < packs;
      if (gather) {
        const WT *row = table + (size_t)tok * p.k + 4 * j;
        x[m] = in ? make_float4((float)row[0], (float)row[1], (float)row[2], (float)row[3]) : make_float4(0, 0, 0, 0);
      } else {
        x[m] = in ? reinterpret_cast<const float4 *>(src)[j] : make_float4(0, 0, 0, 0);
      }
      x2[m] = (in && p.pro_mode == FK_PRO_SILU_MUL) ? reinterpret_cast<const float4 *>(src2)[j]
                                                     : make_float4(0, 0, 0, 0);
      g[m] = (in && p.has_gamma && (p.pro_mode == FK_PRO_RMSNORM || p.pro_mode == FK_PRO_GATHER_RMSNORM))
                 ? reinterpret_cast<const float4 *>(gamma)[j % (p.seg / 4)]
                 : make_float4(1, 1, 1, 1);
    }
  }

  // The anchors' input row into `xs`: gathered rows times the factor, SiLU·mul,
  // or RMSNorm (one segment, the row) of them; a barrier after.
  __device__ __forceinline__ void finish(float *xs, float *slots, const fk_step_gemv_params &p) {
    const uint32_t packs = p.k / 4;
    const bool gather = p.pro_mode == FK_PRO_GATHER || p.pro_mode == FK_PRO_GATHER_RMSNORM;
#pragma unroll
    for (int m = 0; m < NPK; m++) {
      if (gather) {
        x[m].x = x[m].x * p.gfactor;
        x[m].y = x[m].y * p.gfactor;
        x[m].z = x[m].z * p.gfactor;
        x[m].w = x[m].w * p.gfactor;
      } else if (p.pro_mode == FK_PRO_SILU_MUL) {
        x[m] = make_float4(fk::silu_mul(x[m].x, x2[m].x), fk::silu_mul(x[m].y, x2[m].y),
                           fk::silu_mul(x[m].z, x2[m].z), fk::silu_mul(x[m].w, x2[m].w));
      }
    }
    if (p.pro_mode == FK_PRO_RMSNORM || p.pro_mode == FK_PRO_GATHER_RMSNORM) {
      float acc = 0.0f;
#pragma unroll
      for (int m = 0; m < NPK; m++) {
        if (threadIdx.x + m * blockDim.x < packs) {
          acc = acc + x[m].x * x[m].x;
          acc = acc + x[m].y * x[m].y;
          acc = acc + x[m].z * x[m].z;
          acc = acc + x[m].w * x[m].w;
        }
      }
      const float total = fk::block_reduce<false>(acc, slots);
      const float scale = fk::rsqrt_once(total / (float)p.seg + p.eps);
#pragma unroll
      for (int m = 0; m < NPK; m++) {
        float o[4] = {x[m].x * scale, x[m].y * scale, x[m].z * scale, x[m].w * scale};
        if (p.has_gamma) {
          o[0] = o[0] * g[m].x;
          o[1] = o[1] * g[m].y;
          o[2] = o[2] * g[m].z;
          o[3] = o[3] * g[m].w;
        }
        if (p.factor != 1.0f) {
#pragma unroll
          for (int e = 0; e < 4; e++) o[e] = o[e] * p.factor;
        }
        x[m] = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
#pragma unroll
    for (int m = 0; m < NPK; m++) {
      const uint32_t j = threadIdx.x + m * blockDim.x;
      if (j < packs) reinterpret_cast<float4 *>(xs)[j] = x[m];
    }
    __syncthreads();
  }
};

// A GEMV step's threadgroups are persistent: the grid is what fits on the
// device at once, each threadgroup makes the anchors' input row once (its
// prologue) and its wavefronts then take row blocks of R rows in turn, block
// b, b + (all wavefronts), ...  The anchors' rows are numbered one after
// another.  While a wavefront computes a block, the first PF packs of its next
// block are already loading; its first block's packs load before the prologue
// runs, since weights don't depend on it.
template <typename WT, int P, int R, int PF>
__device__ __forceinline__ void step_gemv_body(const WT *__restrict__ w0, const WT *__restrict__ w1,
                                               const WT *__restrict__ w2, float *__restrict__ y0,
                                               float *__restrict__ y1, float *__restrict__ y2,
                                               const float *__restrict__ src, const float *__restrict__ src2,
                                               const float *__restrict__ gamma, const WT *__restrict__ table,
                                               const uint32_t *__restrict__ token, const float *__restrict__ res,
                                               const WT *__restrict__ res_table, const uint32_t *__restrict__ res_token,
                                               float *__restrict__ epi_out, const fk_step_gemv_params &p) {
  __shared__ float xs[FK_STEP_MAX_K];
  __shared__ float slots[16];
  constexpr int C = P / 4;
  constexpr int U = P * sizeof(WT) / 16;
  const uint32_t k = p.k;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t waves = blockDim.x / FK_WAVE;
  const uint32_t total_waves = gridDim.x * waves;
  const uint32_t packs = k / P;
  // Row blocks: anchor a's rows are blocks [first_group[a], first_group[a + 1]).
  const uint32_t blocks = p.first_group[p.n_anchors];

  // Where block b's rows are: its anchor, and the W rows of its R rows.
  auto locate = [&](uint32_t b, uint32_t &a, uint32_t &row0, const WT *(&wr)[R]) {
    a = fk::anchor_of(b, p);
    row0 = (b - fk::pick3(a, p.first_group[0], p.first_group[1], p.first_group[2])) * R;
    const uint32_t n = fk::pick3(a, p.rows[0], p.rows[1], p.rows[2]);
    const WT *wa = fk::pick3(a, w0, w1, w2);
#pragma unroll
    for (int q = 0; q < R; q++) wr[q] = wa + (size_t)min(row0 + q, n - 1) * k;
  };
  auto prefetch = [&](const WT *(&wr)[R], uint4 (&pre)[PF][R][U], bool live) {
#pragma unroll
    for (int it = 0; it < PF; it++) {
      const uint32_t j = lane + it * FK_WAVE;
#pragma unroll
      for (int q = 0; q < R; q++)
#pragma unroll
        for (int u = 0; u < U; u++)
          pre[it][q][u] = (live && j < packs) ? reinterpret_cast<const uint4 *>(wr[q] + (size_t)j * P)[u]
                                              : make_uint4(0, 0, 0, 0);
    }
  };

  uint32_t b = blockIdx.x * waves + threadIdx.x / FK_WAVE;
  uint32_t a, row0;
  const WT *wr[R];
  uint4 cur[PF][R][U];
  Prologue<WT, FK_STEP_MAX_K / (4 * 512)> pro;
  pro.load(src, src2, gamma, table, token, p);
  locate(b < blocks ? b : 0, a, row0, wr);
  prefetch(wr, cur, b < blocks);
  pro.finish(xs, slots, p);
  const uint32_t rtok = (p.epi_mode == FK_EPI_ADD_GATHER) ? min(res_token[0], p.table_rows - 1) : 0;

  for (; b < blocks; b += total_waves) {
    const uint32_t nb = b + total_waves;
    uint32_t na = 0, nrow0 = 0;
    const WT *nwr[R];
    uint4 nxt[PF][R][U];
    locate(nb < blocks ? nb : b, na, nrow0, nwr);
    prefetch(nwr, nxt, nb < blocks);

    // The block's rows, in the reference GEMV's order.
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
      if (j < packs) consume(j, cur[it]);
    }
#pragma unroll 4
    for (uint32_t j = lane + PF * FK_WAVE; j < packs; j += FK_WAVE) {
      uint4 wv4[R][U];
#pragma unroll
      for (int q = 0; q < R; q++)
#pragma unroll
        for (int u = 0; u < U; u++) wv4[q][u] = reinterpret_cast<const uint4 *>(wr[q] + (size_t)j * P)[u];
      consume(j, wv4);
    }
    const uint32_t n = fk::pick3(a, p.rows[0], p.rows[1], p.rows[2]);
    float *ya = fk::pick3(a, y0, y1, y2);
#pragma unroll
    for (int q = 0; q < R; q++) {
      float t = acc[q][0];
#pragma unroll
      for (int c = 1; c < C; c++) t = t + acc[q][c];
      t = fk::wave_sum(t);
      const uint32_t row = row0 + q;
      if (lane == 0 && row < n) {
        if (p.store_tile) ya[row] = t;
        if (p.epi_mode == FK_EPI_ADD_STORED) {
          epi_out[row] = res[row] + t;
        } else if (p.epi_mode == FK_EPI_ADD_GATHER) {
          epi_out[row] = fk::gathered(res_table, rtok, n, row, p.gfactor) + t;
        }
      }
    }
    a = na;
    row0 = nrow0;
#pragma unroll
    for (int q = 0; q < R; q++) wr[q] = nwr[q];
#pragma unroll
    for (int it = 0; it < PF; it++)
#pragma unroll
      for (int q = 0; q < R; q++)
#pragma unroll
        for (int u = 0; u < U; u++) cur[it][q][u] = nxt[it][q][u];
  }
}

// Buffers in binding order, then the parameter struct.
#define FK_STEP_GEMV_ENTRY(NAME, WT, P, R, PF)                                                                      \
  extern "C" __global__ void __launch_bounds__(512)                                                                 \
      NAME(const WT *__restrict__ w0, const WT *__restrict__ w1, const WT *__restrict__ w2, float *__restrict__ y0, \
           float *__restrict__ y1, float *__restrict__ y2, const float *__restrict__ src,                          \
           const float *__restrict__ src2, const float *__restrict__ gamma, const WT *__restrict__ table,           \
           const uint32_t *__restrict__ token, const float *__restrict__ res, const WT *__restrict__ res_table,     \
           const uint32_t *__restrict__ res_token, float *__restrict__ epi_out, fk_step_gemv_params p) {           \
    step_gemv_body<WT, P, R, PF>(w0, w1, w2, y0, y1, y2, src, src2, gamma, table, token, res, res_table, res_token, \
                                 epi_out, p);                                                                       \
  }

FK_STEP_GEMV_ENTRY(fk_step_gemv_f16_r1, _Float16, 8, 1, 4)
FK_STEP_GEMV_ENTRY(fk_step_gemv_f16_r2, _Float16, 8, 2, 4)
FK_STEP_GEMV_ENTRY(fk_step_gemv_f16_r4, _Float16, 8, 4, 2)
FK_STEP_GEMV_ENTRY(fk_step_gemv_f16_r1p8, _Float16, 8, 1, 8)
FK_STEP_GEMV_ENTRY(fk_step_gemv_f32_r1, float, 4, 1, 4)

// GEMV steps of a known input width: every row's weights in registers.
//
// A wavefront takes ROWS consecutive rows (numbered across the anchors) and
// the input width is 64 * P * PPL, so lane l's packs are l, l + 64, ... (PPL
// of them) of each row.  The wavefront issues all ROWS * PPL of its 16-byte
// weight loads when it starts, before the prologue: the whole matrix is
// requested at once and the prologue runs under the loads.  The input row
// lives in dynamic LDS (k floats); with PPL <= 4 each lane keeps its x packs
// in registers for all its rows.  Each row's lane totals are reduced across
// the wavefront together at the end, ROWS independent pairwise trees.
// Same order, same bits as step_gemv_body.
template <typename WT, int P, int ROWS, int PPL>
__device__ __forceinline__ void step_gemv_resident(const WT *__restrict__ w0, const WT *__restrict__ w1,
                                                   const WT *__restrict__ w2, float *__restrict__ y0,
                                                   float *__restrict__ y1, float *__restrict__ y2,
                                                   const float *__restrict__ src, const float *__restrict__ src2,
                                                   const float *__restrict__ gamma, const WT *__restrict__ table,
                                                   const uint32_t *__restrict__ token, const float *__restrict__ res,
                                                   const WT *__restrict__ res_table,
                                                   const uint32_t *__restrict__ res_token, float *__restrict__ epi_out,
                                                   const fk_step_gemv_params &p) {
  extern __shared__ float xs[];
  __shared__ float slots[16];
  constexpr int C = P / 4;
  constexpr int U = P * sizeof(WT) / 16;
  constexpr bool XREG = PPL <= 4;
  const uint32_t k = p.k;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t total = p.first_group[p.n_anchors];  // rows, all anchors
  const uint32_t row_first = (blockIdx.x * (blockDim.x / FK_WAVE) + threadIdx.x / FK_WAVE) * ROWS;

  Prologue<WT, FK_STEP_MAX_K / (4 * 512)> pro;
  pro.load(src, src2, gamma, table, token, p);
  uint32_t anc[ROWS], lrow[ROWS];
  uint4 w[ROWS][PPL][U];
#pragma unroll
  for (int q = 0; q < ROWS; q++) {
    const uint32_t r = row_first + q;
    const uint32_t a = fk::anchor_of(r, p);
    anc[q] = a;
    lrow[q] = r - fk::pick3(a, p.first_group[0], p.first_group[1], p.first_group[2]);
    const bool live = r < total;
    const WT *wr = fk::pick3(a, w0, w1, w2) + (size_t)(live ? lrow[q] : 0) * k;
#pragma unroll
    for (int it = 0; it < PPL; it++)
#pragma unroll
      for (int u = 0; u < U; u++)
        w[q][it][u] = live ? reinterpret_cast<const uint4 *>(wr + (size_t)(lane + it * FK_WAVE) * P)[u]
                           : make_uint4(0, 0, 0, 0);
  }

  pro.finish(xs, slots, p);
  if (row_first >= total) return;

  float xr[XREG ? PPL : 1][XREG ? P : 1];
  if (XREG) {
#pragma unroll
    for (int it = 0; it < PPL; it++)
#pragma unroll
      for (int e = 0; e < P; e++) xr[XREG ? it : 0][XREG ? e : 0] = xs[(lane + it * FK_WAVE) * P + e];
  }
  float t[ROWS];
#pragma unroll
  for (int q = 0; q < ROWS; q++) {
    float acc[C];
#pragma unroll
    for (int c = 0; c < C; c++) acc[c] = 0.0f;
#pragma unroll
    for (int it = 0; it < PPL; it++) {
      float xv[P];
      if (XREG) {
#pragma unroll
        for (int e = 0; e < P; e++) xv[e] = xr[XREG ? it : 0][XREG ? e : 0];
      } else {
#pragma unroll
        for (int e = 0; e < P; e++) xv[e] = xs[(lane + it * FK_WAVE) * P + e];
      }
      float wv[P];
      fk::unpack<P>(w[q][it], wv, WT{});
#pragma unroll
      for (int c = 0; c < C; c++) {
        float p0 = xv[4 * c] * wv[4 * c];
        float p1 = xv[4 * c + 1] * wv[4 * c + 1];
        float p2 = xv[4 * c + 2] * wv[4 * c + 2];
        float p3 = xv[4 * c + 3] * wv[4 * c + 3];
        acc[c] = acc[c] + ((p0 + p1) + (p2 + p3));
      }
    }
    float tq = acc[0];
#pragma unroll
    for (int c = 1; c < C; c++) tq = tq + acc[c];
    t[q] = tq;
  }
  // The wavefront sums of all ROWS rows, level by level.
#pragma unroll
  for (int m = 1; m < FK_WAVE; m <<= 1) {
    float o[ROWS];
#pragma unroll
    for (int q = 0; q < ROWS; q++) o[q] = __shfl_xor(t[q], m);
#pragma unroll
    for (int q = 0; q < ROWS; q++) t[q] = t[q] + o[q];
  }
  if (lane == 0) {
    const uint32_t rtok = (p.epi_mode == FK_EPI_ADD_GATHER) ? min(res_token[0], p.table_rows - 1) : 0;
#pragma unroll
    for (int q = 0; q < ROWS; q++) {
      if (row_first + q >= total) break;
      const uint32_t a = anc[q];
      const uint32_t row = lrow[q];
      if (p.store_tile) fk::pick3(a, y0, y1, y2)[row] = t[q];
      if (p.epi_mode == FK_EPI_ADD_STORED) {
        epi_out[row] = res[row] + t[q];
      } else if (p.epi_mode == FK_EPI_ADD_GATHER) {
        epi_out[row] = fk::gathered(res_table, rtok, fk::pick3(a, p.rows[0], p.rows[1], p.rows[2]), row, p.gfactor) + t[q];
      }
    }
  }
}

#define FK_STEP_GEMV_RESIDENT(NAME, WT, P, ROWS, PPL)                                                             \
  extern "C" __global__ void __launch_bounds__(512)                                                                 \
      NAME(const WT *__restrict__ w0, const WT *__restrict__ w1, const WT *__restrict__ w2, float *__restrict__ y0, \
           float *__restrict__ y1, float *__restrict__ y2, const float *__restrict__ src,                          \
           const float *__restrict__ src2, const float *__restrict__ gamma, const WT *__restrict__ table,           \
           const uint32_t *__restrict__ token, const float *__restrict__ res, const WT *__restrict__ res_table,     \
           const uint32_t *__restrict__ res_token, float *__restrict__ epi_out, fk_step_gemv_params p) {           \
    step_gemv_resident<WT, P, ROWS, PPL>(w0, w1, w2, y0, y1, y2, src, src2, gamma, table, token, res, res_table,   \
                                         res_token, epi_out, p);                                                    \
  }

// f16 weights, k = 2048 (PPL 4) and k = 8192 (PPL 16).
FK_STEP_GEMV_RESIDENT(fk_step_gemv_f16_k2048_r1, _Float16, 8, 1, 4)
FK_STEP_GEMV_RESIDENT(fk_step_gemv_f16_k2048_r2, _Float16, 8, 2, 4)
FK_STEP_GEMV_RESIDENT(fk_step_gemv_f16_k2048_r4, _Float16, 8, 4, 4)
FK_STEP_GEMV_RESIDENT(fk_step_gemv_f16_k2048_r8, _Float16, 8, 8, 4)
FK_STEP_GEMV_RESIDENT(fk_step_gemv_f16_k8192_r1, _Float16, 8, 1, 16)
FK_STEP_GEMV_RESIDENT(fk_step_gemv_f16_k8192_r2, _Float16, 8, 2, 16)

// KV stores ----------------------------------------------------------------

namespace fk {

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

struct fk_step_store_params {
  uint32_t n_stores;    // 1 or 2
  uint32_t rope[2];     // store j's value is RoPE'd first
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t length;      // the ring's positions
  uint32_t slots;       // the ring's sequences
  uint32_t rotated;     // pairs turned
  uint32_t rope_rows;   // positions the RoPE table holds
  uint32_t cache_bf16;  // the caches round to bf16 (else f16)
};

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

// Attention ----------------------------------------------------------------

#define FK_ATTN_MAX_SPLIT 128
#define FK_ATTN_MAX_GROUP 8
#define FK_ATTN_MAX_DIM 64
#define FK_ATTN_THREADS 512
#define FK_ATTN_WAVES (FK_ATTN_THREADS / FK_WAVE)
// A key row in LDS: 64 halves and 8 of padding (144 bytes), so that lanes
// reading 16 bytes of consecutive rows hit distinct banks.
#define FK_ATTN_KROW (FK_ATTN_MAX_DIM + 8)

struct fk_step_attend_params {
  uint32_t heads;
  uint32_t kv_heads;
  uint32_t head_dim;  // a multiple of 8, at most 64
  uint32_t length;    // the ring's positions
  uint32_t slots;
  uint32_t splits;    // threadgroups per kv head
  uint32_t split;     // positions a split covers: split t is [t split, (t + 1) split); 64 or 128
  uint32_t rope;      // q is RoPE'd first
  uint32_t rotated;
  uint32_t rope_rows;
  float scale;        // the attention's scale, rounded once to binary32
  uint32_t window;    // 0: none
  uint32_t cache_bf16;
  uint32_t store;     // the new key and value rows are stored into the caches first
  uint32_t krope;     // the stored key row is RoPE'd first (q's table)
};

namespace fk {

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}

// The wavefront's maximumNumber, every lane, on max_key's integers: within
// rows of 16 lanes by DPP (pairs, quads, halves, rows), then across the four
// rows.  Exact whatever the order.
__device__ __forceinline__ float wave_max_dpp(float x) {
  int v = max_key(x);
  v = max(v, dpp<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max(v, dpp<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max(v, dpp<0x141>(v));  // row_half_mirror
  v = max(v, dpp<0x140>(v));  // row_mirror
  const int a = __builtin_amdgcn_readlane(v, 0);
  const int b = __builtin_amdgcn_readlane(v, 16);
  const int c = __builtin_amdgcn_readlane(v, 32);
  const int d = __builtin_amdgcn_readlane(v, 48);
  return from_max_key(max(max(a, b), max(c, d)));
}

// LDS of one attention threadgroup.
struct AttendLds {
  alignas(16) float qs[FK_ATTN_MAX_GROUP * FK_ATTN_MAX_DIM];
  alignas(16) u32x4 ks[FK_ATTN_MAX_SPLIT * FK_ATTN_KROW / 8];   // later: the runs' weighted values
  alignas(16) u32x4 vs[FK_ATTN_MAX_SPLIT * FK_ATTN_MAX_DIM / 8];
  alignas(16) float wt[FK_ATTN_MAX_SPLIT * FK_ATTN_MAX_GROUP];  // [position][head]
  alignas(16) float pm[FK_ATTN_MAX_GROUP * 2];  // per head, the maxima of the split's 64-position halves
  alignas(16) float pl[FK_ATTN_WAVES * FK_ATTN_MAX_GROUP];     // the runs' weight sums
};

// Threadgroup (kv head g, split t) of 512 threads.  G, D, S, CB: the
// group's query heads, the head dimension, the split's positions and the
// caches' bf16-ness when known at compile time (0, 0, 0, -1: read from the
// parameters).
//
// Store (if asked): the threadgroup whose split holds the position stores kv
// head g's new key row (RoPE'd if asked) and value row at the ring index
// ((s * kvHeads + g) * length + pos mod length) * headDim, rounded to the
// cache's type (Graph.hs:138-143) — what the plan's store step does for that
// head — and takes the rounded rows as that position's key and value.  No
// other position of the ring maps to that index (the gate holds attention to
// what the ring holds), so no other threadgroup reads it.
//
// Attend: for each query head h of the group and each position r of the
// split, score = (sum over i in order of q_i k_i) * scale; the head's maximum
// over the split (exact whatever the order); the weights exp(score - max),
// binary64's rounded once.  The weights' sum and the weighted sum of the
// values over 8 runs of split/8 positions (wavefront w's run w), each in
// order of position from +0, then the runs' sums in order.  Stored as
// partials: per (head, split) [max, sum, acc[head_dim]].
template <uint32_t G, uint32_t D, uint32_t S, int CB>
__device__ __forceinline__ void attend_split(AttendLds &sh, const float *__restrict__ q,
                                             const float *__restrict__ knew, const float *__restrict__ vnew,
                                             uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                             const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot,
                                             const float *__restrict__ rope, float *__restrict__ partials,
                                             const fk_step_attend_params &p) {
  constexpr uint32_t T = FK_ATTN_THREADS;
  constexpr uint32_t HPT = FK_ATTN_MAX_GROUP * FK_ATTN_MAX_SPLIT / T;  // heads a thread scores, at most
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  const uint32_t g = blockIdx.x / p.splits;
  const uint32_t t = blockIdx.x % p.splits;
  const uint32_t group = G ? G : p.heads / p.kv_heads;
  const uint32_t d = D ? D : p.head_dim;
  const uint32_t split = S ? S : p.split;
  const uint32_t half = d / 2;
  const uint32_t pos = position[0];
  const uint32_t sraw = slot[0];
  const uint32_t s = sraw < p.slots ? sraw : 0;
  const bool bf16 = CB >= 0 ? CB != 0 : p.cache_bf16 != 0;
  // Positions [first, pos], this split's part of them.
  const uint32_t first = (p.window && pos + 1 > p.window) ? pos + 1 - p.window : 0;
  const uint32_t lo = max(first, t * split);
  const uint32_t hi = min(pos + 1, (t + 1) * split);
  const uint32_t n = hi > lo ? hi - lo : 0;
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  const bool stores = p.store && sraw < p.slots && lo <= pos && pos < hi;
  uint16_t *ksh = reinterpret_cast<uint16_t *>(sh.ks);
  const uint16_t *vsh = reinterpret_cast<const uint16_t *>(sh.vs);

  // Loads, in the order their results are needed (a wavefront's loads
  // complete in order): the query rows with their RoPE partners and
  // cosines, the new rows, then the split's keys and values, 16 bytes a load.
  float qx = 0.0f, qp = 0.0f, qc = 1.0f, qn = 0.0f;
  if (tid < group * d) {
    const float *head = q + (size_t)(g * group + tid / d) * d;
    const uint32_t j = tid % d;
    const uint32_t i = j < half ? j : j - half;
    qx = head[j];
    if (p.rope && i < p.rotated) {
      qp = head[j < half ? j + half : j - half];
      qc = cs[2 * i];
      qn = cs[2 * i + 1];
    }
  }
  float kx = 0.0f, kp = 0.0f, kcs = 1.0f, ksn = 0.0f, vx = 0.0f;
  if (stores && tid < d) {
    const float *head = knew + (size_t)g * d;
    const uint32_t j = tid;
    const uint32_t i = j < half ? j : j - half;
    kx = head[j];
    if (p.krope && i < p.rotated) {
      kp = head[j < half ? j + half : j - half];
      kcs = cs[2 * i];
      ksn = cs[2 * i + 1];
    }
    vx = vnew[(size_t)g * d + j];
  }
  const uint32_t per_row = d / 8;
  const uint32_t chunks = n * per_row;
  const size_t base = ((size_t)s * p.kv_heads + g) * p.length;
  // Ring index of row r: (lo + r) mod length, where r < n <= length.
  const uint32_t ring0 = lo % p.length;
  u32x4 kr[2], vr[2];
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint32_t e = tid + m * T;
    kr[m] = vr[m] = u32x4{0u, 0u, 0u, 0u};
    if (e < chunks) {
      uint32_t ring = ring0 + e / per_row;
      ring = ring >= p.length ? ring - p.length : ring;
      const size_t at = (base + ring) * d + 8 * (e % per_row);
      kr[m] = *reinterpret_cast<const u32x4 *>(kc + at);
      vr[m] = *reinterpret_cast<const u32x4 *>(vc + at);
    }
  }

  // The query rows, RoPE'd as rope_elem does, and the tile into LDS.
  if (tid < group * d) {
    const uint32_t j = tid % d;
    const uint32_t i = j < half ? j : j - half;
    float v = qx;
    if (p.rope && i < p.rotated) v = j < half ? qx * qc - qp * qn : qx * qc + qp * qn;
    sh.qs[tid] = v;
  }
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint32_t e = tid + m * T;
    if (e < chunks) {
      const uint32_t r = e / per_row;
      const uint32_t c8 = e % per_row;
      sh.ks[r * (FK_ATTN_KROW / 8) + c8] = kr[m];
      sh.vs[r * per_row + c8] = vr[m];
    }
  }
  __syncthreads();
  if (stores && tid < d) {
    const uint32_t j = tid;
    const uint32_t i = j < half ? j : j - half;
    float k = kx;
    if (p.krope && i < p.rotated) k = j < half ? kx * kcs - kp * ksn : kx * kcs + kp * ksn;
    const uint16_t kh = narrow_cache(k, bf16);
    const uint16_t vh = narrow_cache(vx, bf16);
    const size_t at = (base + pos % p.length) * d + j;
    kc[at] = kh;
    vc[at] = vh;
    ksh[(pos - lo) * FK_ATTN_KROW + j] = kh;
    reinterpret_cast<uint16_t *>(sh.vs)[(pos - lo) * d + j] = vh;
  }
  __syncthreads();

  // Scores: thread (r, hs) takes position r of the split for the heads hs,
  // hs + 512/split: its key row read once, 16 bytes at a time.  Each
  // wavefront holds 64 positions of its heads: their maximum by DPP.
  const uint32_t nh = T / split;
  const uint32_t r = tid % split;
  const uint32_t hs = tid / split;
  const uint32_t halfk = r / FK_WAVE;
  float sc[HPT];
  {
    float kf[FK_ATTN_MAX_DIM];
#pragma unroll
    for (uint32_t c8 = 0; c8 < FK_ATTN_MAX_DIM / 8; c8++) {
      u32x4 kk = u32x4{0u, 0u, 0u, 0u};
      if (c8 < per_row && r < n) kk = sh.ks[r * (FK_ATTN_KROW / 8) + c8];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        kf[8 * c8 + 2 * j] = widen_cache((uint16_t)(kk[j] & 0xFFFFu), bf16);
        kf[8 * c8 + 2 * j + 1] = widen_cache((uint16_t)(kk[j] >> 16), bf16);
      }
    }
#pragma unroll
    for (uint32_t a = 0; a < HPT; a++) {
      const uint32_t h = hs + a * nh;
      sc[a] = -__builtin_inff();
      if (h < group && r < n) {
        const float4 *qh = reinterpret_cast<const float4 *>(sh.qs + h * d);
        float dot = 0.0f;
#pragma unroll
        for (uint32_t c4 = 0; c4 < FK_ATTN_MAX_DIM / 4; c4++) {
          if (c4 < d / 4) {
            const float4 qq = qh[c4];
            dot = dot + qq.x * kf[4 * c4];
            dot = dot + qq.y * kf[4 * c4 + 1];
            dot = dot + qq.z * kf[4 * c4 + 2];
            dot = dot + qq.w * kf[4 * c4 + 3];
          }
        }
        sc[a] = dot * p.scale;
      }
    }
#pragma unroll
    for (uint32_t a = 0; a < HPT; a++) {
      const uint32_t h = hs + a * nh;
      if (h < group) {
        const float m = wave_max_dpp(sc[a]);
        if (lane == 0) sh.pm[h * 2 + halfk] = m;
      }
    }
  }
  __syncthreads();
  // The weights exp(score - max), the head's maximum the larger of its halves'.
#pragma unroll
  for (uint32_t a = 0; a < HPT; a++) {
    const uint32_t h = hs + a * nh;
    if (h < group && r < n) {
      const float m = split > FK_WAVE ? max_number(sh.pm[h * 2], sh.pm[h * 2 + 1]) : sh.pm[h * 2];
      sh.wt[r * FK_ATTN_MAX_GROUP + h] = exp_once(sc[a] - m);
    }
  }
  __syncthreads();
  // Wavefront w's run of positions, lane i's dimension, every head at once.
  {
    const uint32_t run = split / FK_ATTN_WAVES;
    const uint32_t u0 = wave * run;
    const uint32_t u1 = min(u0 + run, n);
    float l[FK_ATTN_MAX_GROUP], acc[FK_ATTN_MAX_GROUP];
#pragma unroll
    for (int h = 0; h < FK_ATTN_MAX_GROUP; h++) l[h] = acc[h] = 0.0f;
    if (lane < d) {
      for (uint32_t u = u0; u < u1; u++) {
        const float v = widen_cache(vsh[u * d + lane], bf16);
        const float4 w0 = *reinterpret_cast<const float4 *>(sh.wt + u * FK_ATTN_MAX_GROUP);
        const float4 w1 = group > 4 ? *reinterpret_cast<const float4 *>(sh.wt + u * FK_ATTN_MAX_GROUP + 4)
                                    : float4{0.0f, 0.0f, 0.0f, 0.0f};
        const float w[FK_ATTN_MAX_GROUP] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int h = 0; h < FK_ATTN_MAX_GROUP; h++) {
          if ((uint32_t)h < group) {
            l[h] = l[h] + w[h];
            acc[h] = acc[h] + w[h] * v;
          }
        }
      }
    }
    __syncthreads();  // the keys are no longer read: their LDS holds the runs' sums
    float *pacc = reinterpret_cast<float *>(sh.ks);  // [wave][head][dim]
    if (lane < d) {
#pragma unroll
      for (int h = 0; h < FK_ATTN_MAX_GROUP; h++)
        if ((uint32_t)h < group) pacc[(wave * FK_ATTN_MAX_GROUP + h) * FK_ATTN_MAX_DIM + lane] = acc[h];
    }
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < FK_ATTN_MAX_GROUP; h++)
        if ((uint32_t)h < group) sh.pl[wave * FK_ATTN_MAX_GROUP + h] = l[h];
    }
    __syncthreads();
    if (tid < group * d) {
      const uint32_t h = tid / d;
      const uint32_t i = tid % d;
      float lt = 0.0f;
      float at = 0.0f;
#pragma unroll
      for (int w = 0; w < FK_ATTN_WAVES; w++) {
        lt = lt + sh.pl[w * FK_ATTN_MAX_GROUP + h];
        at = at + pacc[(w * FK_ATTN_MAX_GROUP + h) * FK_ATTN_MAX_DIM + i];
      }
      float *o = partials + ((size_t)(g * group + h) * p.splits + t) * (d + 2);
      if (i == 0) {
        o[0] = split > FK_WAVE ? max_number(sh.pm[h * 2], sh.pm[h * 2 + 1]) : sh.pm[h * 2];
        o[1] = lt;
      }
      o[2 + i] = at;
    }
  }
}

}  // namespace fk

extern "C" __global__ void __launch_bounds__(FK_ATTN_THREADS)
    fk_step_attend(const float *__restrict__ q, const float *__restrict__ knew, const float *__restrict__ vnew,
                   uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                   const uint32_t *__restrict__ slot, const float *__restrict__ rope, float *__restrict__ partials,
                   fk_step_attend_params p) {
  __shared__ fk::AttendLds sh;
  const uint32_t group = p.heads / p.kv_heads;
  if (group == 4 && p.head_dim == 64 && p.split == 128 && !p.cache_bf16)
    fk::attend_split<4, 64, 128, 0>(sh, q, knew, vnew, kc, vc, position, slot, rope, partials, p);
  else if (group == 4 && p.head_dim == 64 && p.split == 64 && !p.cache_bf16)
    fk::attend_split<4, 64, 64, 0>(sh, q, knew, vnew, kc, vc, position, slot, rope, partials, p);
  else
    fk::attend_split<0, 0, 0, -1>(sh, q, knew, vnew, kc, vc, position, slot, rope, partials, p);
}

struct fk_step_combine_params {
  uint32_t heads;
  uint32_t head_dim;
  uint32_t splits;  // at most 256
};

// Threadgroup per head: M the largest of the splits' maxima (exact whatever
// the order), the splits' weights w_t = exp(max_t - M) binary64's rounded
// once, then thread i: out = (sum_t acc_t[i] w_t) / (sum_t l_t w_t), both sums
// in split order, sixteen splits' loads in flight at a time.
extern "C" __global__ void __launch_bounds__(FK_STEP_THREADS)
    fk_step_combine(const float *__restrict__ partials, float *__restrict__ out, fk_step_combine_params p) {
  __shared__ float w[256];
  __shared__ float top;
  const uint32_t h = blockIdx.x;
  const uint32_t stride = p.head_dim + 2;
  const float *ph = partials + (size_t)h * p.splits * stride;
  if (threadIdx.x < FK_WAVE) {
    float m = -__builtin_inff();
    for (uint32_t t = threadIdx.x; t < p.splits; t += FK_WAVE) m = fk::max_number(m, ph[t * stride]);
    m = fk::wave_max(m);
    if (threadIdx.x == 0) top = m;
  }
  __syncthreads();
  for (uint32_t t = threadIdx.x; t < p.splits; t += blockDim.x) w[t] = fk::exp_once(ph[t * stride] - top);
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < p.head_dim; i += blockDim.x) {
    float l = 0.0f;
    float acc = 0.0f;
    for (uint32_t t0 = 0; t0 < p.splits; t0 += 16) {
      float lv[16], av[16];
#pragma unroll
      for (int j = 0; j < 16; j++) {
        lv[j] = av[j] = 0.0f;
        if (t0 + j < p.splits) {
          lv[j] = ph[(t0 + j) * stride + 1];
          av[j] = ph[(t0 + j) * stride + 2 + i];
        }
      }
#pragma unroll
      for (int j = 0; j < 16; j++) {
        if (t0 + j < p.splits) {
          l = l + lv[j] * w[t0 + j];
          acc = acc + av[j] * w[t0 + j];
        }
      }
    }
    out[(size_t)h * p.head_dim + i] = acc / l;
  }
}

struct fk_step_argmax_params {
  uint32_t n;
};

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
