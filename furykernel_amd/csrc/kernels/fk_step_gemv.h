// fk_step_gemv.h — the GEMV step of a planned decode step
// (src/FuryKernel/Program/Plan.hs:17-31): one launch whose threadgroups make
// the anchors' input row (the recomputed chain: RMSNorm of a stored or gathered
// row, a gathered row, SiLU·mul of two stored rows, or a stored row), then take
// blocks of the anchors' output rows — each row y_j = sum_i W[j, i] x_i in the
// reference GEMV's order at SIMD width 64, split 1 — and run the step's
// epilogue on the tile.
//
// Layout in HBM: each anchor's W is [rows, k] row-major (`out_in`,
// src/FuryKernel/Program/Build.hs:175-176), f16 or f32; x, y and the epilogue
// rows are f32.
//
// Work split: the anchors' rows are numbered one after another; a block is R
// consecutive rows (or, for the SiLU·mul epilogue, rows j .. j + R/2 - 1 of
// both anchors, so a wavefront holds gate_j and up_j together).  A wavefront
// takes blocks b, b + (all wavefronts), ...; lane l holds packs l, l + 64, ...
// (KPL of them at most, 16 bytes each) of each of its rows.  A block's weight
// loads are all issued at once, and with DB the next block's are issued
// before the current block is computed, so a wavefront keeps two blocks in
// flight.  The prologue's loads go out first, the first block's weights right
// after them: the prologue's arithmetic and its one barrier run while the
// weights stream in.
//
// Order (the bits): per row, lane l's pack elements four to a chain
// ((x0 w0 + x1 w1) + (x2 w2 + x3 w3)), each chain summed over the lane's packs
// in order, the lane's chains added in order, then the pairwise wavefront sum
// (test/Test/FuryKernel/Gemv.hs:16-23,131-191).  RMSNorm's sum of squares in
// tgReduceSum's order with the launch's threads (src/FuryKernel/Reduce.hs:55-85).
#pragma once

#include "fk_common.h"
#include "fk_gemv.h"

#define FK_GEMV_MAX_K 8192
// Threads of every GEMV step launch: a compile-time constant, since reading
// the launch's size costs the kernel a load from the dispatch packet.
#define FK_GEMV_THREADS 512

namespace fk {

// A weight or table element as binary32 (exact for every type here).
__device__ __forceinline__ float to_float(float x) { return x; }
__device__ __forceinline__ float to_float(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_float(bf16_t x) { return __uint_as_float((uint32_t)x.bits << 16); }
template <typename WT>
__device__ __forceinline__ float widen_half(uint16_t h) {
  if constexpr (__is_same(WT, bf16_t)) return __uint_as_float((uint32_t)h << 16);
  else return widen_f16(h);
}

// An anchor's pointer or count by index, without indexing an array: a
// dynamically indexed array of kernel pointers would lose their address space
// (its loads would become flat loads, which wait with LDS traffic).
template <typename T>
__device__ __forceinline__ T pick3(uint32_t a, T x0, T x1, T x2) {
  return a == 0 ? x0 : (a == 1 ? x1 : x2);
}

// Where slot q of block b is: its anchor, its row in the anchor, and whether
// it exists.
template <int R>
struct Block {
  uint32_t anchor[R];
  uint32_t row[R];
  bool live[R];

  __device__ __forceinline__ void locate(uint32_t b, const fk_step_gemv_params &p) {
    const bool paired = p.epi_mode == FK_EPI_SILU_MUL;
    const uint32_t total = p.first_row[p.n_anchors];
#pragma unroll
    for (int q = 0; q < R; q++) {
      if (paired && R == 1) {
        // One row a block: blocks 2j and 2j + 1 are row j of the first
        // anchor and of the second, held by a wavefront and the next.
        anchor[q] = b & 1u;
        row[q] = b >> 1;
        live[q] = b < p.blocks && row[q] < p.rows[0];
      } else if (paired) {
        constexpr uint32_t H = R / 2 > 0 ? R / 2 : 1;
        anchor[q] = (uint32_t)q < H ? 0u : 1u;
        row[q] = b * H + ((uint32_t)q % H);
        live[q] = b < p.blocks && row[q] < p.rows[0];
      } else {
        const uint32_t g = b * R + q;
        const uint32_t a = (p.n_anchors > 1 && g >= p.first_row[1] ? 1u : 0u) +
                           (p.n_anchors > 2 && g >= p.first_row[2] ? 1u : 0u);
        anchor[q] = a;
        row[q] = g - pick3(a, p.first_row[0], p.first_row[1], p.first_row[2]);
        live[q] = b < p.blocks && g < total;
      }
    }
  }
};

}  // namespace fk

// Loads a wavefront issues are waited for in the order it issued them, and
// the compiler counts them only through straight-line code: so every load here
// is unconditional (its address clamped into the buffer, its value replaced
// by zero where it lies outside the row), the prologue and epilogue modes are
// template parameters, and the block loop alternates between two named
// buffers rather than copying one into the other.  Each use then waits for its
// own loads only, never for the ones issued after them.

namespace fk {

// A block's weights: R rows of KPL 16-byte packs a lane, loaded non-temporal
// (a step streams each weight once).
template <typename WT, int P, int R, int KPL>
__device__ __forceinline__ void issue_block(uint4 (&dst)[R][KPL], const Block<R> &blk, const WT *__restrict__ w0,
                                            const WT *__restrict__ w1, const WT *__restrict__ w2, uint32_t k,
                                            uint32_t packs, uint32_t lane, const fk_step_gemv_params &p) {
#pragma unroll
  for (int q = 0; q < R; q++) {
    const uint32_t a = blk.anchor[q];
    const uint32_t n = pick3(a, p.rows[0], p.rows[1], p.rows[2]);
    const WT *wr = pick3(a, w0, w1, w2) + (size_t)min(blk.row[q], n - 1) * k;
#pragma unroll
    for (int it = 0; it < KPL; it++) {
      const uint32_t j = lane + it * FK_WAVE;
      dst[q][it] = load16<true>(wr + (size_t)min(j, packs - 1) * P);
    }
  }
}

}  // namespace fk

// One wavefront's block loop.  WT: weight element; P: elements a 16-byte pack
// holds; R: rows a block; KPL: packs a lane holds of a row (k <= 64 P KPL);
// DB: the next block's weights in flight while a block is computed (else
// issued after it); PRO, EPI: the prologue and epilogue modes.
template <typename WT, int P, int R, int KPL, bool DB, uint32_t PRO, uint32_t EPI>
__device__ __forceinline__ void step_gemv(const WT *__restrict__ w0, const WT *__restrict__ w1, const WT *__restrict__ w2,
                                          float *__restrict__ y0, float *__restrict__ y1, float *__restrict__ y2,
                                          const float *__restrict__ src, const float *__restrict__ src2,
                                          const float *__restrict__ gamma, const WT *__restrict__ table,
                                          const uint32_t *__restrict__ token, const float *__restrict__ res,
                                          const WT *__restrict__ res_table, const uint32_t *__restrict__ res_token,
                                          float *__restrict__ epi_out, unsigned long long *__restrict__ arg,
                                          const fk_step_gemv_params &p) {
  static_assert(P * sizeof(WT) == 16, "a pack is one 16-byte load");
  static_assert(EPI != FK_EPI_SILU_MUL || R % 2 == 0 || R == 1, "the SiLU·mul epilogue pairs rows");
  // The SiLU·mul epilogue at one row a block: a wavefront's row and its
  // neighbour's meet in LDS (each threadgroup's wavefronts run the same
  // number of blocks, one barrier a block).
  constexpr bool PAIR1 = EPI == FK_EPI_SILU_MUL && R == 1;
  constexpr int C = P / 4;
  // The prologue's packs of 4 a thread holds, at most, with the 512 threads
  // every launch of these kernels has.
  constexpr int NPK = KPL * P / 32 > 0 ? KPL * P / 32 : 1;
  constexpr bool GATHER = PRO == FK_PRO_GATHER || PRO == FK_PRO_GATHER_RMSNORM;
  constexpr bool NORM = PRO == FK_PRO_RMSNORM || PRO == FK_PRO_GATHER_RMSNORM;
  constexpr bool SILU = PRO == FK_PRO_SILU_MUL;
  constexpr bool COMBINE = PRO == FK_PRO_COMBINE;
  // The combine prologue's splits at most (its loads are straight-line).
  constexpr uint32_t CS = 8;
  constexpr bool RESIDUAL = EPI == FK_EPI_ADD_STORED || EPI == FK_EPI_ADD_GATHER;
  // The input row (normalized, for the norm prologues) in LDS transposed to
  // the lanes' packs: chunk c (4 elements) of lane l's pack it is float4 (it C + c) 64 + l,
  // so a wavefront reads a chunk of all its lanes' packs with one conflict-free
  // 16-byte load a lane.  XT float4s: 64 P KPL / 4 a row.
  constexpr uint32_t XT = 64 * P * KPL / 4;
  extern __shared__ float4 lds4[];  // xt[XT]
  __shared__ float slots[16];
  __shared__ unsigned long long bests[16];
  __shared__ float pairv[PAIR1 ? 2 : 1][PAIR1 ? 16 : 1];  // PAIR1: each wavefront's row, by block parity
  float4 *xt = lds4;
  const uint32_t k = p.k;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  constexpr uint32_t waves = FK_GEMV_THREADS / FK_WAVE;
  const uint32_t total_waves = gridDim.x * waves;
  const uint32_t packs = k / P;
  const uint32_t packs4 = k / 4;
  const bool has_gamma = NORM && p.has_gamma;
  const float gfactor = p.gfactor;
  const float eps = p.eps;
  const float factor = p.factor;
  const uint32_t blocks = p.blocks;
  // Where pack-of-4 j of the row (elements 4j .. 4j + 3) lives in xt.
  auto xt_at = [](uint32_t j) -> uint32_t {
    const uint32_t pk = j / C;
    return ((pk / FK_WAVE) * C + j % C) * FK_WAVE + pk % FK_WAVE;
  };

  // Prologue loads: thread t's packs of 4, t, t + T, ... (tgReduceSum's order).
  const uint32_t tok = GATHER ? min(token[0], p.table_rows - 1) : 0u;
  float4 xa[NPK], xb[NPK], ga[NPK];
  // The combine prologue: pack-of-4 j of the row is head h's dimensions
  // i .. i + 3; its splits' accumulators (float4 each) and (max, sum) pairs.
  float4 ca[COMBINE ? NPK : 1][COMBINE ? CS : 1];
  float2 cst[COMBINE ? NPK : 1][COMBINE ? CS : 1];
#pragma unroll
  for (int m = 0; m < NPK; m++) {
    const uint32_t j = min(tid + m * FK_GEMV_THREADS, packs4 - 1);
    if constexpr (COMBINE) {
      const uint32_t e = 4 * j;
      const uint32_t hd = p.head_dim;
      const uint32_t h = e / hd, i = e % hd;
      const uint32_t heads = k / hd;
      const float *st = src + (size_t)heads * p.splits * hd + (size_t)h * p.splits * 2;
#pragma unroll
      for (uint32_t tt = 0; tt < CS; tt++) {
        const uint32_t tc = min(tt, p.splits - 1);
        ca[m][tt] = *reinterpret_cast<const float4 *>(src + ((size_t)h * p.splits + tc) * hd + i);
        cst[m][tt] = *reinterpret_cast<const float2 *>(st + 2 * tc);
      }
      xa[m] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else if constexpr (GATHER) {
      const WT *row = table + (size_t)tok * k + 4 * j;
      if constexpr (sizeof(WT) == 2) {
        const uint2 h = *reinterpret_cast<const uint2 *>(row);
        xa[m] = make_float4(fk::widen_half<WT>((uint16_t)(h.x & 0xFFFFu)), fk::widen_half<WT>((uint16_t)(h.x >> 16)),
                            fk::widen_half<WT>((uint16_t)(h.y & 0xFFFFu)), fk::widen_half<WT>((uint16_t)(h.y >> 16)));
      } else {
        const float4 v = *reinterpret_cast<const float4 *>(row);
        xa[m] = v;
      }
    } else {
      xa[m] = reinterpret_cast<const float4 *>(src)[j];
    }
    if constexpr (SILU) xb[m] = reinterpret_cast<const float4 *>(src2 + p.src2_off)[j];
    // A norm without gains has a row of ones bound here (the product is then
    // not taken), so the load is unconditional.
    if constexpr (NORM) ga[m] = reinterpret_cast<const float4 *>(gamma)[j];
  }
  const uint32_t rtok = EPI == FK_EPI_ADD_GATHER ? min(res_token[0], p.table_rows - 1) : 0u;

  // The first block's weights.
  uint32_t b = blockIdx.x * waves + wave;
  fk::Block<R> ba, bb;
  uint4 wa[R][KPL], wb[DB ? R : 1][DB ? KPL : 1];
  ba.locate(b, p);
  fk::issue_block<WT, P, R, KPL>(wa, ba, w0, w1, w2, k, packs, lane, p);

  // The prologue's arithmetic: the row (and the gains) into LDS, each wave's
  // sum of squares into its slot; one barrier.  Slots of xt past the row hold
  // zeros.
  float acc = 0.0f;
#pragma unroll
  for (int m = 0; m < NPK; m++) {
    const uint32_t j = tid + m * FK_GEMV_THREADS;
    float4 v = xa[m];
    if constexpr (GATHER) {
      v.x = v.x * gfactor;
      v.y = v.y * gfactor;
      v.z = v.z * gfactor;
      v.w = v.w * gfactor;
    }
    if constexpr (COMBINE) {
      // The combine kernel's arithmetic (fk_step_combine): the splits' largest
      // maximum, their weights exp(m_t - top) binary64's rounded once, then in
      // split order from +0: l += l_t w_t, acc += acc_t w_t; x = acc / l.
      int tk = fk::max_key(-__builtin_inff());
#pragma unroll
      for (uint32_t tt = 0; tt < CS; tt++)
        if (tt < p.splits) tk = max(tk, fk::max_key(cst[m][tt].x));
      const float top = fk::from_max_key(tk);
      float l = 0.0f;
      float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t tt = 0; tt < CS; tt++) {
        if (tt < p.splits) {
          const float w = fk::exp_once(cst[m][tt].x - top);
          const float lw = cst[m][tt].y * w;
          l = l + lw;
          a4[0] = a4[0] + ca[m][tt].x * w;
          a4[1] = a4[1] + ca[m][tt].y * w;
          a4[2] = a4[2] + ca[m][tt].z * w;
          a4[3] = a4[3] + ca[m][tt].w * w;
        }
      }
      v = make_float4(a4[0] / l, a4[1] / l, a4[2] / l, a4[3] / l);
    }
    if constexpr (SILU) {
      const uint32_t act = p.act;
      v = make_float4(fk::act_mul(v.x, xb[m].x, act), fk::act_mul(v.y, xb[m].y, act),
                      fk::act_mul(v.z, xb[m].z, act), fk::act_mul(v.w, xb[m].w, act));
    }
    if (j < packs4) {
      if constexpr (NORM) {
        acc = acc + v.x * v.x;
        acc = acc + v.y * v.y;
        acc = acc + v.z * v.z;
        acc = acc + v.w * v.w;
      }
      xt[xt_at(j)] = v;
    } else if (j < XT) {
      xt[xt_at(j)] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
  if constexpr (NORM) {
    const float s = fk::wave_sum(acc);
    if (lane == 0) slots[wave] = s;
  }
  __syncthreads();
  // tgReduceSum's last steps, in every wavefront: lane l folds slots l, l + 64,
  // ... from -0, then the wavefront sum.
  float scale = 1.0f;
  if constexpr (NORM) {
    const float sl = slots[min(lane, waves - 1)];
    const float t = -0.0f + (lane < waves ? sl : -0.0f);
    scale = fk::rsqrt_once(fk::wave_sum(t) / (float)p.seg + eps);
    // The normalized row, once: each thread's own packs of 4 to ((x scale)
    // gamma) factor (both products made, one kept by a select), written over
    // their place; one more barrier.  Every block then reads the row as it
    // stands instead of normalizing it again.
#pragma unroll
    for (int m = 0; m < NPK; m++) {
      const uint32_t j = tid + m * FK_GEMV_THREADS;
      if (j < packs4) {
        const float4 v = xt[xt_at(j)];
        float e[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
        const float gg[4] = {ga[m].x, ga[m].y, ga[m].z, ga[m].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float eg = e[q] * gg[q];
          e[q] = has_gamma ? eg : e[q];
          const float ef = e[q] * factor;
          e[q] = factor != 1.0f ? ef : e[q];
        }
        xt[xt_at(j)] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
    __syncthreads();
  }
  // Chunk c of lane l's pack it of the anchors' input row.
  auto xin4 = [&](int it, int c) -> float4 { return xt[(it * C + c) * FK_WAVE + lane]; };
  uint64_t best = 0;
  uint32_t turn = 0;  // PAIR1: the blocks run so far
  // Block `blk`'s rows from the weights `w`: the residuals loaded first (lane q
  // holds slot q's), then (with DB) the next block's weights issued into `wn`,
  // then the block computed, reduced and its epilogue run.
  auto run = [&](const fk::Block<R> &blk, const uint4 (&w)[R][KPL], fk::Block<R> &bn, uint4 (&wn)[R][KPL],
                 uint32_t nb) {
    float resv = 0.0f;
    if constexpr (RESIDUAL) {
      uint32_t a = blk.anchor[0], r = blk.row[0];
#pragma unroll
      for (int q = 1; q < R; q++)
        if (lane == (uint32_t)q) a = blk.anchor[q], r = blk.row[q];
      const uint32_t n = fk::pick3(a, p.rows[0], p.rows[1], p.rows[2]);
      if constexpr (EPI == FK_EPI_ADD_STORED) {
        resv = res[min(r, n - 1)];
      } else {
        resv = fk::to_float(res_table[(size_t)rtok * n + min(r, n - 1)]) * gfactor;
      }
    }
    if constexpr (DB) {
      bn.locate(nb, p);
      fk::issue_block<WT, P, R, KPL>(wn, bn, w0, w1, w2, k, packs, lane, p);
    }

    float t[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      float a[C];
#pragma unroll
      for (int c = 0; c < C; c++) a[c] = 0.0f;
#pragma unroll
      for (int it = 0; it < KPL; it++) {
        const uint32_t j = lane + it * FK_WAVE;
        float wv[P];
        const uint4 u[1] = {w[q][it]};
        fk::unpack<P>(u, wv, WT{});
        float xv[P];
#pragma unroll
        for (int c = 0; c < C; c++) {
          const float4 x4 = xin4(it, c);
          xv[4 * c] = x4.x;
          xv[4 * c + 1] = x4.y;
          xv[4 * c + 2] = x4.z;
          xv[4 * c + 3] = x4.w;
        }
        // A pack past the row adds +0 in place of its products (the lane never
        // visits it): exact, since a chain that starts at +0 is never -0.
        const bool in = j < packs;
#pragma unroll
        for (int c = 0; c < C; c++) {
          const float p0 = xv[4 * c] * wv[4 * c];
          const float p1 = xv[4 * c + 1] * wv[4 * c + 1];
          const float p2 = xv[4 * c + 2] * wv[4 * c + 2];
          const float p3 = xv[4 * c + 3] * wv[4 * c + 3];
          const float ps = (p0 + p1) + (p2 + p3);
          a[c] = a[c] + (in ? ps : 0.0f);
        }
      }
      float s = a[0];
#pragma unroll
      for (int c = 1; c < C; c++) s = s + a[c];
      t[q] = s;
    }
    fk::wave_sums<R>(t);

    if constexpr (PAIR1) {
      // Row j of the first anchor (even wavefront) and of the second (the
      // odd one next to it): both tiles stored, then act(first) · second
      // by the even wavefront, from its partner's value in LDS.
      const uint32_t a = blk.anchor[0], r = blk.row[0];
      if (lane == 0) {
        if (blk.live[0] && p.store_tile) fk::pick3(a, y0, y1, y2)[r] = t[0];
        pairv[turn & 1][wave] = t[0];
      }
      __syncthreads();
      if (lane == 0 && blk.live[0] && a == 0) epi_out[r] = fk::act_mul(t[0], pairv[turn & 1][wave + 1], p.act);
      turn++;
      return;
    }
    // Epilogue: slot q's stores by lane q.
#pragma unroll
    for (int q = 0; q < R; q++) {
      if (blk.live[q]) {
        float capped = 0.0f;
        if constexpr (EPI == FK_EPI_SOFTCAP) capped = fk::softcap(t[q], p.cap);
        if constexpr (EPI == FK_EPI_ARGMAX) {
          const uint64_t key = fk::argmax_key(t[q], blk.row[q]);
          best = key > best ? key : best;
        }
        if constexpr (EPI == FK_EPI_SOFTCAP) {
          const uint64_t key = fk::argmax_key(capped, blk.row[q]);
          best = key > best ? key : best;
        }
        if (lane == (uint32_t)q) {
          const uint32_t a = blk.anchor[q];
          const uint32_t r = blk.row[q];
          if (p.store_tile) fk::pick3(a, y0, y1, y2)[r] = t[q];
          if constexpr (RESIDUAL) epi_out[r] = resv + t[q];
          if constexpr (EPI == FK_EPI_SILU_MUL) {
            if (q < R / 2) epi_out[r] = fk::act_mul(t[q], t[(q + R / 2) % R], p.act);
          }
          if constexpr (EPI == FK_EPI_SOFTCAP) epi_out[r] = capped;
        }
      }
    }
  };

  if constexpr (DB) {
    while (b < blocks) {
      run(ba, wa, bb, wb, b + total_waves);
      b += total_waves;
      if (b >= blocks) break;
      run(bb, wb, ba, wa, b + total_waves);
      b += total_waves;
    }
  } else if constexpr (PAIR1) {
    // Every wavefront of the threadgroup runs as many blocks as its first
    // (a barrier a block): a block past the last is run dead, its loads
    // clamped into the weights.
    uint32_t b0 = blockIdx.x * waves;
    while (b0 < blocks) {
      run(ba, wa, bb, wa, 0);
      b += total_waves;
      b0 += total_waves;
      if (b0 >= blocks) break;
      ba.locate(b, p);
      fk::issue_block<WT, P, R, KPL>(wa, ba, w0, w1, w2, k, packs, lane, p);
    }
  } else {
    while (b < blocks) {
      run(ba, wa, bb, wa, 0);
      b += total_waves;
      if (b >= blocks) break;
      ba.locate(b, p);
      fk::issue_block<WT, P, R, KPL>(wa, ba, w0, w1, w2, k, packs, lane, p);
    }
  }
  if constexpr (EPI == FK_EPI_ARGMAX || EPI == FK_EPI_SOFTCAP) {
    // The threadgroup's largest key into its own slot of `arg`; the token
    // launch takes the largest of the slots (a softcap with no slots folds no
    // argmax).
    if (lane == 0) bests[wave] = best;
    __syncthreads();
    if (tid == 0 && blockIdx.x < p.arg_slots) {
      unsigned long long m = 0;
      for (uint32_t w = 0; w < waves; w++) m = bests[w] > m ? bests[w] : m;
      arg[blockIdx.x] = m;
    }
  }
}

// Buffers in binding order, then the parameter struct.
#define FK_STEP_GEMV(NAME, WT, P, R, KPL, DB, PRO, EPI)                                                                \
  extern "C" __global__ void __launch_bounds__(FK_GEMV_THREADS)                                                     \
      NAME(const WT *__restrict__ w0, const WT *__restrict__ w1, const WT *__restrict__ w2, float *__restrict__ y0, \
           float *__restrict__ y1, float *__restrict__ y2, const float *__restrict__ src,                          \
           const float *__restrict__ src2, const float *__restrict__ gamma, const WT *__restrict__ table,           \
           const uint32_t *__restrict__ token, const float *__restrict__ res, const WT *__restrict__ res_table,     \
           const uint32_t *__restrict__ res_token, float *__restrict__ epi_out,                                    \
           unsigned long long *__restrict__ arg, fk_step_gemv_params p) {                                           \
    step_gemv<WT, P, R, KPL, DB, PRO, EPI>(w0, w1, w2, y0, y1, y2, src, src2, gamma, table, token, res,          \
                                           res_table, res_token, epi_out, arg, p);                                  \
  }

// Every prologue with the epilogues a shape takes: entries named
// <shape>_p<prologue>_e<epilogue>.
#define FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, PRO)    \
  FK_STEP_GEMV(NAME##_p##PRO##_e0, WT, P, R, KPL, DB, PRO, 0) \
  FK_STEP_GEMV(NAME##_p##PRO##_e1, WT, P, R, KPL, DB, PRO, 1) \
  FK_STEP_GEMV(NAME##_p##PRO##_e2, WT, P, R, KPL, DB, PRO, 2) \
  FK_STEP_GEMV(NAME##_p##PRO##_e4, WT, P, R, KPL, DB, PRO, 4) \
  FK_STEP_GEMV(NAME##_p##PRO##_e5, WT, P, R, KPL, DB, PRO, 5)
#define FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, PRO) \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, PRO)         \
  FK_STEP_GEMV(NAME##_p##PRO##_e3, WT, P, R, KPL, DB, PRO, 3)
#define FK_STEP_GEMV_SHAPE(NAME, WT, P, R, KPL, DB) \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, 0)      \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, 1)      \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, 2)      \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, 3)      \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, 4)      \
  FK_STEP_GEMV_PRO(NAME, WT, P, R, KPL, DB, 5)
#define FK_STEP_GEMV_SHAPE_PAIRS(NAME, WT, P, R, KPL, DB) \
  FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, 0)          \
  FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, 1)          \
  FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, 2)          \
  FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, 3)          \
  FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, 4)          \
  FK_STEP_GEMV_PAIRS(NAME, WT, P, R, KPL, DB, 5)

// f16 weights: k up to 2048 (4 packs a lane) in blocks of 1 or 2 rows; k up to
// 8192 (16 packs a lane), one row a block.  A block's loads are issued when the
// block before it is done: the memory's parallelism comes from the resident
// wavefronts, each with one block in flight.
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_f16_k2048_r1, _Float16, 8, 1, 4, false)
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_f16_k2048_r2, _Float16, 8, 2, 4, false)
FK_STEP_GEMV_SHAPE(fk_step_gemv_f16_k8192_r1, _Float16, 8, 1, 16, false)
// bf16 weights (the reference builder's): the f16 shapes.
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_bf16_k2048_r1, fk::bf16_t, 8, 1, 4, false)
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_bf16_k2048_r2, fk::bf16_t, 8, 2, 4, false)
FK_STEP_GEMV_SHAPE(fk_step_gemv_bf16_k8192_r1, fk::bf16_t, 8, 1, 16, false)
// f32 weights: k up to 256 and 1024.
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_f32_k256_r1, float, 4, 1, 1, false)
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_f32_k256_r2, float, 4, 2, 1, false)
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_f32_k1024_r1, float, 4, 1, 4, false)
FK_STEP_GEMV_SHAPE_PAIRS(fk_step_gemv_f32_k1024_r2, float, 4, 2, 4, false)

// The greedy token from the folded argmax: the largest of the threadgroups'
// keys (exact whatever the order), its index the complement of the key's low
// word; with `advance`, the next decode step's token is this one and its
// position `step` on.  One wavefront.
extern "C" __global__ void __launch_bounds__(FK_WAVE)
    fk_step_token(const unsigned long long *__restrict__ arg, uint32_t *__restrict__ out,
                  uint32_t *__restrict__ token, uint32_t *__restrict__ position, fk_step_token_params p) {
  const uint32_t lane = threadIdx.x;
  unsigned long long m = 0;
  for (uint32_t i = lane; i < p.slots; i += FK_WAVE) m = arg[i] > m ? arg[i] : m;
  for (int s = 1; s < FK_WAVE; s <<= 1) {
    const unsigned long long o = __shfl_xor(m, s);
    m = o > m ? o : m;
  }
  if (lane == 0) {
    const uint32_t t = 0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull);
    out[0] = t;
    if (p.advance) {
      token[0] = t;
      position[0] = (position[0] + p.step) % p.context;
    }
  }
}
