// fk_prefill.h — the kernels around the prefill GEMM, for a step of many rows
// (the rows of one or more sequences, each a contiguous run of consecutive
// positions):
//
//   fk_prefill_gather      x = embed[token] · factor, f32 rows
//   fk_prefill_norm_pack   RMSNorm of f32 rows into f16 in the tile layout
//                          (the GEMM's A)
//   fk_prefill_land        staged k and v rows landed in the ring
//   fk_prefill_rope_store  q RoPE'd into f16 rows; k RoPE'd and v stored into
//                          the caches at each row's position
//   fk_prefill_softcap     a softcap over rows (the head's, before the argmax)
//   fk_prefill_argmax      the greedy token of each row
//   fk_prefill_argmax_keys the same from the keys the head's GEMM folded in
//
// (The causal attention between them, fk_prefill_attend_g*, is fk_attend.h:
// a code object of its own.)
//
// Semantics follow src/FuryKernel/Program/Eval.hs (RmsNorm :292-305, Rope
// :634-645, KvStore :331-349, Attend :351-380, Gather :382-392) per row; the
// f16 roundings of the GEMM operands are this target's (the f16 bar).
#pragma once

#include "fk_common.h"
#include "fk_layout.h"
#include "fk_mfma.h"

// x[r] = table[tokens[r]] · factor.  One wave a row, 4 columns a lane at a
// time; rows × width f32 out.  A token past the table reads its last row
// (the host refuses such tokens before they get here).

extern "C" __global__ void __launch_bounds__(256) fk_prefill_gather(const void *__restrict__ table,
                                                                    const uint32_t *__restrict__ tokens,
                                                                    float *__restrict__ x,
                                                                    fk_prefill_gather_params p) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / FK_WAVE;
  if (row >= p.rows) return;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint32_t t = min(tokens[row], p.table_rows - 1);
  float *out = x + (size_t)row * p.width;
  for (uint32_t c = 4 * lane; c < p.width; c += 4 * FK_WAVE) {
    float4 v;
    if (p.table_f16) {
      const uint2 h = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(table) + (size_t)t * p.width + c);
      v = make_float4(fk::widen_f16(h.x & 0xffffu), fk::widen_f16(h.x >> 16), fk::widen_f16(h.y & 0xffffu),
                      fk::widen_f16(h.y >> 16));
    } else {
      v = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(table) + (size_t)t * p.width + c);
    }
    *reinterpret_cast<float4 *>(out + c) =
        make_float4(v.x * p.factor, v.y * p.factor, v.z * p.factor, v.w * p.factor);
  }
}

// y = f16(x · (mean(x²) + eps)^-1/2 · g · factor) in the tile layout of a
// [rows, width] matrix.  One wave a row: a pass for the sum of squares (a
// lane's units, then the wave's tree), a pass (the row now in L2) for the
// output, one 16-byte unit of 8 columns a lane at a time.

extern "C" __global__ void __launch_bounds__(256) fk_prefill_norm_pack(const float *__restrict__ x,
                                                                       const float *__restrict__ gamma,
                                                                       uint16_t *__restrict__ y,
                                                                       fk_prefill_norm_params p) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / FK_WAVE;
  if (row >= p.rows) return;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const float *xr = x + (size_t)row * p.width;
  const uint32_t units = p.width / 8;
  float ss = 0.0f;
  for (uint32_t u = lane; u < units; u += FK_WAVE) {
    const float4 a = *reinterpret_cast<const float4 *>(xr + 8 * u);
    const float4 b = *reinterpret_cast<const float4 *>(xr + 8 * u + 4);
    ss += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) + ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
  }
  ss = fk::wave_sum(ss);
  const float s = fk::rsqrt_once(ss / (float)p.width + p.eps);
  for (uint32_t u = lane; u < units; u += FK_WAVE) {
    const float4 a = *reinterpret_cast<const float4 *>(xr + 8 * u);
    const float4 b = *reinterpret_cast<const float4 *>(xr + 8 * u + 4);
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float g[8] = {1, 1, 1, 1, 1, 1, 1, 1};
    if (p.has_gamma) {
      const float4 ga = *reinterpret_cast<const float4 *>(gamma + 8 * u);
      const float4 gb = *reinterpret_cast<const float4 *>(gamma + 8 * u + 4);
      g[0] = ga.x; g[1] = ga.y; g[2] = ga.z; g[3] = ga.w; g[4] = gb.x; g[5] = gb.y; g[6] = gb.z; g[7] = gb.w;
    }
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t lo = fk::to_f16(v[2 * e] * s * g[2 * e] * p.factor);
      const uint32_t hi = fk::to_f16(v[2 * e + 1] * s * g[2 * e + 1] * p.factor);
      h[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4 *>(y + fk::tile_offset(row, 8 * u, p.width)) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

// The same in one pass for rows of exactly 512 U columns: a lane holds its
// U units of 8 in registers between the sum and the output, so each row is
// read from HBM once.
template <int U>
__device__ __forceinline__ void norm_pack_held(const float *__restrict__ x, const float *__restrict__ gamma,
                                               uint16_t *__restrict__ y, const fk_prefill_norm_params &p) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / FK_WAVE;
  if (row >= p.rows) return;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  constexpr uint32_t width = 512 * U;
  const float *xr = x + (size_t)row * width;
  // The row and the gains are loaded together, so that the gains' round
  // trip is not added after the row's sum.
  float4 a[U], b[U], ga[U], gb[U];
#pragma unroll
  for (int t = 0; t < U; t++) {
    a[t] = *reinterpret_cast<const float4 *>(xr + 8 * (lane + 64 * t));
    b[t] = *reinterpret_cast<const float4 *>(xr + 8 * (lane + 64 * t) + 4);
  }
#pragma unroll
  for (int t = 0; t < U; t++) {
    ga[t] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    gb[t] = ga[t];
    if (p.has_gamma) {
      ga[t] = *reinterpret_cast<const float4 *>(gamma + 8 * (lane + 64 * t));
      gb[t] = *reinterpret_cast<const float4 *>(gamma + 8 * (lane + 64 * t) + 4);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int t = 0; t < U; t++)
    ss += ((a[t].x * a[t].x + a[t].y * a[t].y) + (a[t].z * a[t].z + a[t].w * a[t].w)) +
          ((b[t].x * b[t].x + b[t].y * b[t].y) + (b[t].z * b[t].z + b[t].w * b[t].w));
  ss = fk::wave_sum(ss);
  const float s = fk::rsqrt_once(ss / (float)width + p.eps);
#pragma unroll
  for (int t = 0; t < U; t++) {
    const uint32_t u = lane + 64 * t;
    const float g[8] = {ga[t].x, ga[t].y, ga[t].z, ga[t].w, gb[t].x, gb[t].y, gb[t].z, gb[t].w};
    const float v[8] = {a[t].x, a[t].y, a[t].z, a[t].w, b[t].x, b[t].y, b[t].z, b[t].w};
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
      h[e] = fk::to_f16(v[2 * e] * s * g[2 * e] * p.factor) |
             ((uint32_t)fk::to_f16(v[2 * e + 1] * s * g[2 * e + 1] * p.factor) << 16);
    *reinterpret_cast<uint4 *>(y + fk::tile_offset(row, 8 * u, width)) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

#define FK_NORM_PACK_HELD(W, U)                                                                                 \
  extern "C" __global__ void __launch_bounds__(256) fk_prefill_norm_pack_w##W(                                  \
      const float *__restrict__ x, const float *__restrict__ gamma, uint16_t *__restrict__ y,                   \
      fk_prefill_norm_params p) {                                                                               \
    norm_pack_held<U>(x, gamma, y, p);                                                                          \
  }
FK_NORM_PACK_HELD(512, 1)
FK_NORM_PACK_HELD(1024, 2)
FK_NORM_PACK_HELD(2048, 4)
FK_NORM_PACK_HELD(4096, 8)

// q RoPE'd into f16 rows [rows, heads · d]; k RoPE'd and v into the caches
// ([slots][kv_heads][length][d], f16 or bf16) at (slot, head, position mod
// length).  One threadgroup a row.  The cache stores round as the decode
// step's stores do (narrowF16 / narrowBF16).

// PG: kc and vc are paged pools ([blocks][kv_heads][block_size][d]) and
// `slot` the rows' block tables ([rows][table_len]).
template <bool PG>
__device__ __forceinline__ void prefill_rope_store(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, const uint32_t *__restrict__ position,
                                                   const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                                   uint16_t *__restrict__ qr, uint16_t *__restrict__ kc,
                                                   uint16_t *__restrict__ vc, const fk_prefill_rope_params &p,
                                                   const fk_paging &pg = fk_paging{}) {
  const uint32_t row = blockIdx.x;
  const uint32_t d = p.head_dim;
  const uint32_t pos = position[row];
  // the row's ring slot, or its position's block through its table (both
  // clamped into place); a position past its table stores no k or v, as
  // the decode step's paged store skips it
  const uint32_t sl = PG ? min(slot[(size_t)row * pg.table_len + min(pos / pg.block_size, pg.table_len - 1)],
                               pg.blocks - 1)
                         : min(slot[row], p.slots - 1);
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  const uint32_t qw = p.heads * d, kw = p.kv_heads * d;
  const uint32_t stored = !PG || pos / pg.block_size < pg.table_len ? qw + 2 * kw : qw;
  const float *qx = q + (size_t)row * qw;
  const float *kx = k + (size_t)row * kw;
  const float *vx = v + (size_t)row * kw;
  const bool bf16 = p.cache_bf16 != 0;
  for (uint32_t e = threadIdx.x; e < stored; e += blockDim.x) {
    if (e < qw) {
      qr[(size_t)row * qw + e] = fk::to_f16(fk::rope_elem(qx + (e / d) * d, e % d, d, p.rotated, cs));
    } else {
      const uint32_t f = e < qw + kw ? e - qw : e - qw - kw;
      const uint32_t h = f / d, i = f % d;
      const size_t at = PG        ? (((size_t)sl * p.kv_heads + h) * pg.block_size + pos % pg.block_size) * d + i
                        : p.staged ? ((size_t)row * p.kv_heads + h) * d + i
                                   : (((size_t)sl * p.kv_heads + h) * p.length + pos % p.length) * d + i;
      if (e < qw + kw)
        kc[at] = fk::narrow_cache(fk::rope_elem(kx + h * d, i, d, p.rotated, cs), bf16);
      else
        vc[at] = fk::narrow_cache(vx[f], bf16);
    }
  }
}

extern "C" __global__ void __launch_bounds__(256) fk_prefill_rope_store(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot, const float *__restrict__ rope,
    uint16_t *__restrict__ qr, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, fk_prefill_rope_params p) {
  prefill_rope_store<false>(q, k, v, position, slot, rope, qr, kc, vc, p);
}

// The same storing k and v into paged pools through the rows' block tables.
extern "C" __global__ void __launch_bounds__(256) fk_prefill_rope_store_paged(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const uint32_t *__restrict__ position, const uint32_t *__restrict__ table, const float *__restrict__ rope,
    uint16_t *__restrict__ qr, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    fk_prefill_rope_paged_params p) {
  prefill_rope_store<true>(q, k, v, position, table, rope, qr, kc, vc, p.r, p.g);
}

// Staged rows landed (Plan.hs:41-50): row r's k and v heads, as the caches
// hold them, from the staging rows into the ring at (slot, head, position
// mod length).  One threadgroup a row; a copy of 16-bit elements.
extern "C" __global__ void __launch_bounds__(256) fk_prefill_land(
    const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs, const uint32_t *__restrict__ position,
    const uint32_t *__restrict__ slot, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    fk_prefill_land_params p) {
  const uint32_t row = blockIdx.x;
  const uint32_t kw = p.kv_heads * p.head_dim;
  const uint32_t pos = position[row];
  const uint32_t sl = min(slot[row], p.slots - 1);
  for (uint32_t e = threadIdx.x; e < 2 * kw; e += blockDim.x) {
    const uint32_t f = e < kw ? e : e - kw;
    const uint32_t h = f / p.head_dim, i = f % p.head_dim;
    const size_t at = (((size_t)sl * p.kv_heads + h) * p.length + pos % p.length) * p.head_dim + i;
    if (e < kw)
      kc[at] = ks[(size_t)row * kw + f];
    else
      vc[at] = vs[(size_t)row * kw + f];
  }
}

// A softcap over the logits of every row (src/FuryKernel/Program/Eval.hs:
// 384-390), in place or into another buffer: y = cap tanh(x / cap), as the
// decode step's epilogue computes it.
extern "C" __global__ void __launch_bounds__(256) fk_prefill_softcap(const float *__restrict__ x,
                                                                     float *__restrict__ y,
                                                                     fk_prefill_softcap_params p) {
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < p.count; i += gridDim.x * 256) y[i] = fk::softcap(x[i], p.cap);
}

// The greedy token of each row: the index of its largest logit, the first
// of equals, by the decode step's 64-bit keys (value order, then the
// complement of the index; a NaN at index 0 wins, elsewhere loses:
// src/FuryKernel/Program/Eval.hs:681-685).  One wave a row.
extern "C" __global__ void __launch_bounds__(256) fk_prefill_argmax(const float *__restrict__ x,
                                                                    uint32_t *__restrict__ out,
                                                                    fk_prefill_argmax_params p) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / FK_WAVE;
  if (row >= p.rows) return;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const float *xr = x + (size_t)row * p.width;
  uint64_t best = 0;
  for (uint32_t j = lane; j < p.width; j += FK_WAVE) {
    const uint64_t key = fk::argmax_key(xr[j], j);
    best = key > best ? key : best;
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(best >> 32), s) << 32) |
                           (uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)best, s);
    best = other > best ? other : best;
  }
  if (lane == 0) out[row] = 0xFFFFFFFFu - (uint32_t)best;
}

// The greedy token of each row from the keys fk_gemm_f16_store_keys left,
// `parts` a row (the keys of its columns 128 at a time): their maximum is
// the maximum of every element's key, the fold fk_prefill_argmax makes.  One
// wave a row.
extern "C" __global__ void __launch_bounds__(256) fk_prefill_argmax_keys(const uint64_t *__restrict__ keys,
                                                                         uint32_t *__restrict__ out,
                                                                         fk_prefill_argmax_keys_params p) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / FK_WAVE;
  if (row >= p.rows) return;
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
  const uint64_t *kr = keys + (size_t)row * p.parts;
  uint64_t best = 0;
  for (uint32_t j = lane; j < p.parts; j += FK_WAVE) best = kr[j] > best ? kr[j] : best;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(best >> 32), s) << 32) |
                           (uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)best, s);
    best = other > best ? other : best;
  }
  if (lane == 0) out[row] = 0xFFFFFFFFu - (uint32_t)best;
}
