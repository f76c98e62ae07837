// fk_gemv.h — matrix-vector products in the reference GEMV's order
// (test/Test/FuryKernel/Gemv.hs:5-27,131-191), as wave64 kernels.
//
// y = W x for one row x: W is [n, k] row-major (the `out_in` layout,
// src/FuryKernel/Program/Build.hs:170-176).  A wavefront takes R whole rows:
// lane l visits packs l, l + 64, ... of P consecutive elements (one 16-byte
// load of W per pack), the pack's elements four to a chain
// ((x0 w0 + x1 w1) + (x2 w2 + x3 w3)), each chain its own sum; then the
// lane's chains in order and the pairwise wavefront sum.
//
// That is the reference order at SIMD width 64, split 1.  It is also, bit for
// bit, the CPU target's order at width 32, split 2 (src/FuryKernel/Cpu.hs:73):
// there lane v = 32 q + l of split q visits the same packs v, v + 64, ..., each
// split's 32 lanes sum pairwise, and the combine adds split 0's partial to
// split 1's (src/FuryKernel/Reduce.hs:112-125) — the last step of the width-64
// pairwise tree.
#pragma once

#include "fk_common.h"

namespace fk {

// 16 bytes; NT: a non-temporal load, for data read once (the weights, which
// a step streams past every cache), so that it does not displace the rows
// and partials every threadgroup reads.
template <bool NT>
__device__ __forceinline__ uint4 load16(const void *p) {
  if constexpr (NT) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return uint4{v[0], v[1], v[2], v[3]};
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}

// A pack of P elements of W or x, widened to f32 exactly.
template <int P, bool NT = false>
__device__ __forceinline__ void load_pack(const float *__restrict__ p, float (&out)[P]) {
  static_assert(P % 4 == 0, "f32 packs are float4s");
#pragma unroll
  for (int i = 0; i < P / 4; i++) {
    const uint4 u = load16<NT>(p + 4 * i);
    const float4 v = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
    out[4 * i] = v.x;
    out[4 * i + 1] = v.y;
    out[4 * i + 2] = v.z;
    out[4 * i + 3] = v.w;
  }
}

// A pack of 4 half elements: one 8-byte load.
template <bool NT>
__device__ __forceinline__ uint2 load8(const void *p) {
  if constexpr (NT) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
    return uint2{v[0], v[1]};
  } else {
    return *reinterpret_cast<const uint2 *>(p);
  }
}

template <int P, bool NT = false>
__device__ __forceinline__ void load_pack(const _Float16 *__restrict__ p, float (&out)[P]) {
  if constexpr (P == 4) {
    const uint2 v = load8<NT>(p);
    out[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v.x & 0xFFFFu));
    out[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v.x >> 16));
    out[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y & 0xFFFFu));
    out[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y >> 16));
    return;
  }
  static_assert(P == 4 || P % 8 == 0, "f16 packs are 8- or 16-byte loads");
#pragma unroll
  for (int i = 0; i < P / 8; i++) {
    uint4 v = load16<NT>(p + 8 * i);
    uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; h++) {
      out[8 * i + 2 * h] = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[h] & 0xFFFFu));
      out[8 * i + 2 * h + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[h] >> 16));
    }
  }
}

template <int P, bool NT = false>
__device__ __forceinline__ void load_pack(const bf16_t *__restrict__ p, float (&out)[P]) {
  if constexpr (P == 4) {
    const uint2 v = load8<NT>(p);
    out[0] = __uint_as_float(v.x << 16);
    out[1] = __uint_as_float(v.x & 0xFFFF0000u);
    out[2] = __uint_as_float(v.y << 16);
    out[3] = __uint_as_float(v.y & 0xFFFF0000u);
    return;
  }
  static_assert(P == 4 || P % 8 == 0, "bf16 packs are 8- or 16-byte loads");
#pragma unroll
  for (int i = 0; i < P / 8; i++) {
    uint4 v = load16<NT>(p + 8 * i);
    uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; h++) {
      out[8 * i + 2 * h] = __uint_as_float(words[h] << 16);
      out[8 * i + 2 * h + 1] = __uint_as_float(words[h] & 0xFFFF0000u);
    }
  }
}

template <int P, bool NT = false>
__device__ __forceinline__ void load_pack(const int8_t *__restrict__ p, float (&out)[P]) {
  static_assert(P % 16 == 0, "i8 packs are 16-byte loads");
#pragma unroll
  for (int i = 0; i < P / 16; i++) {
    uint4 v = load16<NT>(p + 16 * i);
    uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int b = 0; b < 16; b++) out[16 * i + b] = (float)(int8_t)(words[b / 4] >> (8 * (b % 4)));
  }
}

// A pack held in registers as 16-byte words, widened to f32 exactly.
template <int P>
__device__ __forceinline__ void unpack(const uint4 (&u)[P / 4], float (&out)[P], float) {
#pragma unroll
  for (int i = 0; i < P / 4; i++) {
    out[4 * i] = __uint_as_float(u[i].x);
    out[4 * i + 1] = __uint_as_float(u[i].y);
    out[4 * i + 2] = __uint_as_float(u[i].z);
    out[4 * i + 3] = __uint_as_float(u[i].w);
  }
}

template <int P>
__device__ __forceinline__ void unpack(const uint4 (&u)[P / 8], float (&out)[P], _Float16) {
#pragma unroll
  for (int i = 0; i < P / 8; i++) {
    const uint32_t words[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
    for (int h = 0; h < 4; h++) {
      out[8 * i + 2 * h] = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[h] & 0xFFFFu));
      out[8 * i + 2 * h + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[h] >> 16));
    }
  }
}

// One 16-byte word of W widened to f32 exactly: 4 f32, 8 f16 or 16 int8.
template <int P>
__device__ __forceinline__ void unpack(const uint4 (&u)[P / 8], float (&out)[P], bf16_t) {
#pragma unroll
  for (int i = 0; i < P / 8; i++) {
    const uint32_t words[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
    for (int h = 0; h < 4; h++) {
      out[8 * i + 2 * h] = __uint_as_float(words[h] << 16);
      out[8 * i + 2 * h + 1] = __uint_as_float(words[h] & 0xFFFF0000u);
    }
  }
}
template <int P>
__device__ __forceinline__ void unpack_w(const uint4 &u, float (&out)[P], float) {
  static_assert(P == 4, "four f32 a word");
  out[0] = __uint_as_float(u.x);
  out[1] = __uint_as_float(u.y);
  out[2] = __uint_as_float(u.z);
  out[3] = __uint_as_float(u.w);
}

template <int P>
__device__ __forceinline__ void unpack_w(const uint4 &u, float (&out)[P], _Float16) {
  static_assert(P == 8, "eight f16 a word");
  const uint32_t words[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int h = 0; h < 4; h++) {
    out[2 * h] = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[h] & 0xFFFFu));
    out[2 * h + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[h] >> 16));
  }
}

template <int P>
__device__ __forceinline__ void unpack_w(const uint4 &u, float (&out)[P], bf16_t) {
  static_assert(P == 8, "eight bf16 a word");
  const uint32_t words[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int h = 0; h < 4; h++) {
    out[2 * h] = __uint_as_float(words[h] << 16);
    out[2 * h + 1] = __uint_as_float(words[h] & 0xFFFF0000u);
  }
}

template <int P>
__device__ __forceinline__ void unpack_w(const uint4 &u, float (&out)[P], int8_t) {
  static_assert(P == 16, "sixteen int8 a word");
  const uint32_t words[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int b = 0; b < 16; b++) out[b] = (float)(int8_t)(words[b / 4] >> (8 * (b % 4)));
}

// R rows of y = W x (times a per-row scale if given) by one wavefront.
template <typename WT, typename XT, int P, int R>
__device__ __forceinline__ void gemv_wave(const WT *__restrict__ w, const XT *__restrict__ x, const float *__restrict__ scale,
                                         float *__restrict__ y, uint32_t n, uint32_t k, uint32_t row0) {
  constexpr int C = P / 4;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t packs = k / P;
  float acc[R][C];
#pragma unroll
  for (int q = 0; q < R; q++)
#pragma unroll
    for (int c = 0; c < C; c++) acc[q][c] = 0.0f;
  // Rows past n read row n - 1 and store nothing: every lane takes part in
  // the wavefront sums.
  const WT *wr[R];
#pragma unroll
  for (int q = 0; q < R; q++) wr[q] = w + (size_t)min(row0 + q, n - 1) * k;
#pragma unroll 4
  for (uint32_t j = lane; j < packs; j += FK_WAVE) {
    float xv[P];
    load_pack<P>(x + (size_t)j * P, xv);
#pragma unroll
    for (int q = 0; q < R; q++) {
      float wv[P];
      load_pack<P, true>(wr[q] + (size_t)j * P, wv);
#pragma unroll
      for (int c = 0; c < C; c++) {
        float p0 = xv[4 * c] * wv[4 * c];
        float p1 = xv[4 * c + 1] * wv[4 * c + 1];
        float p2 = xv[4 * c + 2] * wv[4 * c + 2];
        float p3 = xv[4 * c + 3] * wv[4 * c + 3];
        acc[q][c] = acc[q][c] + ((p0 + p1) + (p2 + p3));
      }
    }
  }
#pragma unroll
  for (int q = 0; q < R; q++) {
    float t = acc[q][0];
#pragma unroll
    for (int c = 1; c < C; c++) t = t + acc[q][c];
    t = wave_sum(t);
    const uint32_t row = row0 + q;
    if (lane == 0 && row < n) y[row] = scale ? t * scale[row] : t;
  }
}

// The same rows and order with every load in flight at once, for rows of at
// most 64 KPL packs: each lane issues all of its packs' 16-byte loads — W's
// first, then x's, the indices clamped into the row so every load is
// unconditional and the compiler keeps them all outstanding — and only then
// computes, packs past the row skipped.  One round trip to memory a
// wavefront, where the loop above waits for each unrolled group of packs in
// turn.  FULL: the row fills every lane's KPL packs (k = 64 KPL P), so no
// pack needs the check.
template <typename WT, typename XT, int P, int R, int KPL, bool FULL>
__device__ __forceinline__ void gemv_wave_inflight(const WT *__restrict__ w, const XT *__restrict__ x,
                                                   const float *__restrict__ scale, float *__restrict__ y,
                                                   uint32_t n, uint32_t k, uint32_t row0) {
  constexpr int C = P / 4;
  constexpr int XW = P * (int)sizeof(XT) / 16;  // 16-byte words of an x pack
  static_assert(P * sizeof(WT) == 16, "a W pack is one 16-byte load");
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t packs = k / P;
  const WT *wr[R];
#pragma unroll
  for (int q = 0; q < R; q++) wr[q] = w + (size_t)min(row0 + q, n - 1) * k;
  uint4 wv[R][KPL], xv[KPL][XW];
#pragma unroll
  for (int it = 0; it < KPL; it++) {
    const uint32_t jc = min(lane + FK_WAVE * (uint32_t)it, packs - 1);
#pragma unroll
    for (int q = 0; q < R; q++) wv[q][it] = load16<true>(wr[q] + (size_t)jc * P);
  }
#pragma unroll
  for (int it = 0; it < KPL; it++) {
    const uint32_t jc = min(lane + FK_WAVE * (uint32_t)it, packs - 1);
#pragma unroll
    for (int u = 0; u < XW; u++) xv[it][u] = reinterpret_cast<const uint4 *>(x + (size_t)jc * P)[u];
  }
  float acc[R][C];
#pragma unroll
  for (int q = 0; q < R; q++)
#pragma unroll
    for (int c = 0; c < C; c++) acc[q][c] = 0.0f;
#pragma unroll
  for (int it = 0; it < KPL; it++) {
    // A pack past the row is computed from the clamped loads and not added:
    // a select, so that no load sits in a branch.
    const bool live = lane + FK_WAVE * (uint32_t)it < packs;
    float xf[P];
    unpack<P>(xv[it], xf, XT{});
#pragma unroll
    for (int q = 0; q < R; q++) {
      float wf[P];
      unpack_w<P>(wv[q][it], wf, WT{});
#pragma unroll
      for (int c = 0; c < C; c++) {
        float p0 = xf[4 * c] * wf[4 * c];
        float p1 = xf[4 * c + 1] * wf[4 * c + 1];
        float p2 = xf[4 * c + 2] * wf[4 * c + 2];
        float p3 = xf[4 * c + 3] * wf[4 * c + 3];
        const float sum = acc[q][c] + ((p0 + p1) + (p2 + p3));
        acc[q][c] = FULL || live ? sum : acc[q][c];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < R; q++) {
    float t = acc[q][0];
#pragma unroll
    for (int c = 1; c < C; c++) t = t + acc[q][c];
    t = wave_sum(t);
    const uint32_t row = row0 + q;
    if (lane == 0 && row < n) y[row] = scale ? t * scale[row] : t;
  }
}

// The int8 weights' full rows (k = 64 KPL 16) with x (f16) staged once a
// threadgroup of T threads in LDS, where every wavefront would otherwise read
// the whole 16 KB x row from memory beside its own 8 KB of weights: the x
// loads first (T into 16-byte chunks), then the rows' weights, then the
// chunks into LDS transposed (chunk u of lane l's pack it at (2 it + u) 64 +
// l, so a wavefront's reads meet distinct banks) and one barrier.  The same
// sums as gemv_wave_inflight: each product of an int8 and an f16 is exact in
// binary32, so a pair's sum p0 + p1 is one fused multiply-add of the second
// product onto the first (one rounding either way), the chain of four
// (p0 + p1) + (p2 + p3).  Every wavefront reaches the barrier: rows past n
// read row n - 1 and store nothing.
template <int T, int R, int KPL>
__device__ __forceinline__ void gemv_i8_xlds(const int8_t *__restrict__ w, const _Float16 *__restrict__ x,
                                             const float *__restrict__ scale, float *__restrict__ y, uint32_t n,
                                             uint32_t row0) {
  constexpr int P = 16, C = 4;
  constexpr uint32_t K = 64 * KPL * P;
  constexpr uint32_t CH = K * 2 / 16;  // x's 16-byte chunks
  constexpr int PER = CH / T;
  static_assert(CH % T == 0, "x's chunks divide among the threads");
  __shared__ uint4 xs[CH];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  uint4 xc[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) xc[i] = reinterpret_cast<const uint4 *>(x)[tid + i * T];
  uint4 wv[R][KPL];
#pragma unroll
  for (int q = 0; q < R; q++) {
    const int8_t *wr = w + (size_t)min(row0 + q, n - 1) * K;
#pragma unroll
    for (int it = 0; it < KPL; it++) wv[q][it] = load16<true>(wr + (size_t)(lane + FK_WAVE * it) * P);
  }
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const uint32_t j = tid + i * T, pack = j / 2;
    xs[((pack / FK_WAVE) * 2 + j % 2) * FK_WAVE + pack % FK_WAVE] = xc[i];
  }
  __syncthreads();
  float acc[R][C];
#pragma unroll
  for (int q = 0; q < R; q++)
#pragma unroll
    for (int c = 0; c < C; c++) acc[q][c] = 0.0f;
#pragma unroll
  for (int it = 0; it < KPL; it++) {
    const uint4 xu[2] = {xs[(2 * it) * FK_WAVE + lane], xs[(2 * it + 1) * FK_WAVE + lane]};
    float xf[P];
    unpack<P>(xu, xf, _Float16{});
#pragma unroll
    for (int q = 0; q < R; q++) {
      float wf[P];
      unpack_w<P>(wv[q][it], wf, int8_t{});
#pragma unroll
      for (int c = 0; c < C; c++) {
        const float s01 = __builtin_fmaf(xf[4 * c + 1], wf[4 * c + 1], xf[4 * c] * wf[4 * c]);
        const float s23 = __builtin_fmaf(xf[4 * c + 3], wf[4 * c + 3], xf[4 * c + 2] * wf[4 * c + 2]);
        acc[q][c] = acc[q][c] + (s01 + s23);
      }
    }
  }
  float t[R];
#pragma unroll
  for (int q = 0; q < R; q++) {
    t[q] = acc[q][0];
#pragma unroll
    for (int c = 1; c < C; c++) t[q] = t[q] + acc[q][c];
  }
  wave_sums<R>(t);
#pragma unroll
  for (int q = 0; q < R; q++) {
    const uint32_t row = row0 + q;
    if (lane == 0 && row < n) y[row] = scale ? t[q] * scale[row] : t[q];
  }
}

}  // namespace fk

// Entry points: a threadgroup of W wavefronts takes W * R consecutive rows;
// rows of at most 64 KPL packs take the all-in-flight form.
// Kernargs: the buffers in binding order, then the parameter struct.

#define FK_GEMV_ENTRY(NAME, WT, XT, P, R, KPL)                                                                 \
  extern "C" __global__ void __launch_bounds__(256) NAME(const WT *__restrict__ w, const XT *__restrict__ x, \
                                                         float *__restrict__ y, fk_gemv_params p) {         \
    const uint32_t row0 = (blockIdx.x * (blockDim.x / FK_WAVE) + threadIdx.x / FK_WAVE) * (R);             \
    if (row0 >= p.n) return;                                                                                 \
    if (p.k / (P) == FK_WAVE * (KPL))                                                                        \
      fk::gemv_wave_inflight<WT, XT, P, R, KPL, true>(w, x, nullptr, y, p.n, p.k, row0);                    \
    else if (p.k / (P) < FK_WAVE * (KPL))                                                                    \
      fk::gemv_wave_inflight<WT, XT, P, R, KPL, false>(w, x, nullptr, y, p.n, p.k, row0);                   \
    else                                                                                                     \
      fk::gemv_wave<WT, XT, P, R>(w, x, nullptr, y, p.n, p.k, row0);                                         \
  }

// The int8 entries: full rows of 64 KPL packs in threadgroups of 256 with x
// staged in LDS (gemv_i8_xlds); other widths and threadgroups by the loop
// form (which keeps the kernel's registers to what the staged form needs,
// so that as many wavefronts as its LDS allows are resident).
#define FK_GEMV_SCALED_ENTRY(NAME, WT, XT, P, R, KPL)                                                      \
  extern "C" __global__ void __launch_bounds__(256)                                                        \
      NAME(const WT *__restrict__ w, const float *__restrict__ scale, const XT *__restrict__ x,            \
           float *__restrict__ y, fk_gemv_params p) {                                                      \
    const uint32_t row0 = (blockIdx.x * (blockDim.x / FK_WAVE) + threadIdx.x / FK_WAVE) * (R);           \
    if (p.k / (P) == FK_WAVE * (KPL) && blockDim.x == 256) {                                               \
      fk::gemv_i8_xlds<256, R, KPL>(w, x, scale, y, p.n, row0);                                            \
      return;                                                                                              \
    }                                                                                                      \
    if (row0 >= p.n) return;                                                                               \
    fk::gemv_wave<WT, XT, P, R>(w, x, scale, y, p.n, p.k, row0);                                           \
  }

// Rows whose width is a multiple of 4 but not of a 16-byte pack (the small
// programs' linear layers): packs of 4 elements, the loop form.
#define FK_GEMV_P4_ENTRY(NAME, WT)                                                                            \
  extern "C" __global__ void __launch_bounds__(256) NAME(const WT *__restrict__ w, const float *__restrict__ x, \
                                                         float *__restrict__ y, fk_gemv_params p) {           \
    const uint32_t row0 = blockIdx.x * (blockDim.x / FK_WAVE) + threadIdx.x / FK_WAVE;                       \
    if (row0 >= p.n) return;                                                                                   \
    fk::gemv_wave<WT, float, 4, 1>(w, x, nullptr, y, p.n, p.k, row0);                                          \
  }
FK_GEMV_P4_ENTRY(fk_gemv_p4_f32, float)
FK_GEMV_P4_ENTRY(fk_gemv_p4_f16, _Float16)
FK_GEMV_P4_ENTRY(fk_gemv_p4_bf16, fk::bf16_t)

// LinearRouted: threadgroup (rank, group) of a rank's groups_per_rank takes
// its W * R rows of the rank's table entry, the id clamped into the table.
#define FK_GEMV_ROUTED_ENTRY(NAME, WT, P, R, KPL)                                                            \
  extern "C" __global__ void __launch_bounds__(256)                                                        \
      NAME(const uint64_t *__restrict__ table, const uint32_t *__restrict__ ids, const float *__restrict__ x, \
           float *__restrict__ y, fk_gemv_routed_params p) {                                               \
    const uint32_t rank = blockIdx.x / p.groups_per_rank;                                                  \
    const uint32_t grp = blockIdx.x % p.groups_per_rank;                                                   \
    const uint32_t row0 = (grp * (blockDim.x / FK_WAVE) + threadIdx.x / FK_WAVE) * (R);                  \
    if (rank >= p.ranks || row0 >= p.n) return;                                                            \
    const uint32_t e = min(ids[rank], p.entries - 1);                                                      \
    const WT *w = reinterpret_cast<const WT *>(table[e]);                                                  \
    const float *xr = x + (p.shared ? (size_t)0 : (size_t)rank * p.k);                                     \
    float *yr = y + (size_t)rank * p.n;                                                                    \
    if (p.k / (P) == FK_WAVE * (KPL))                                                                      \
      fk::gemv_wave_inflight<WT, float, P, R, KPL, true>(w, xr, nullptr, yr, p.n, p.k, row0);             \
    else if (p.k / (P) < FK_WAVE * (KPL))                                                                  \
      fk::gemv_wave_inflight<WT, float, P, R, KPL, false>(w, xr, nullptr, yr, p.n, p.k, row0);            \
    else                                                                                                   \
      fk::gemv_wave<WT, float, P, R>(w, xr, nullptr, yr, p.n, p.k, row0);                                  \
  }

FK_GEMV_ROUTED_ENTRY(fk_gemv_routed_f16_r1, _Float16, 8, 1, 8)
FK_GEMV_ROUTED_ENTRY(fk_gemv_routed_f16_r2, _Float16, 8, 2, 8)
FK_GEMV_ROUTED_ENTRY(fk_gemv_routed_f32_r1, float, 4, 1, 16)
// bf16 tables (the reference builder's `table`, Program/Build.hs:185-186).
FK_GEMV_ROUTED_ENTRY(fk_gemv_routed_bf16_r1, fk::bf16_t, 8, 1, 8)
FK_GEMV_ROUTED_ENTRY(fk_gemv_routed_bf16_r2, fk::bf16_t, 8, 2, 8)

// Packs a lane holds in flight: rows of 4096 f32, 4096 f16 (by one row or
// two) and 8192 int8; wider rows take the loop.
FK_GEMV_ENTRY(fk_gemv_f32_f32_r1, float, float, 4, 1, 16)
FK_GEMV_ENTRY(fk_gemv_f32_f32_r2, float, float, 4, 2, 16)
FK_GEMV_ENTRY(fk_gemv_f32_f32_r4, float, float, 4, 4, 4)
FK_GEMV_ENTRY(fk_gemv_f16_f32_r1, _Float16, float, 8, 1, 8)
FK_GEMV_ENTRY(fk_gemv_f16_f32_r2, _Float16, float, 8, 2, 8)
FK_GEMV_ENTRY(fk_gemv_f16_f32_r4, _Float16, float, 8, 4, 4)
FK_GEMV_SCALED_ENTRY(fk_gemv_i8_f16_r1, int8_t, _Float16, 16, 1, 8)
FK_GEMV_SCALED_ENTRY(fk_gemv_i8_f16_r2, int8_t, _Float16, 16, 2, 8)
FK_GEMV_SCALED_ENTRY(fk_gemv_i8_f16_r4, int8_t, _Float16, 16, 4, 4)
