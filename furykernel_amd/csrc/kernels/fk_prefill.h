// fk_prefill.h — the kernels around the prefill GEMM, for a step of many rows
// (the rows of one or more sequences, each a contiguous run of consecutive
// positions):
//
//   fk_prefill_gather      x = embed[token] · factor, f32 rows
//   fk_prefill_norm_pack   RMSNorm of f32 rows into f16 in the tile layout
//                          (the GEMM's A)
//   fk_prefill_rope_store  q RoPE'd into f16 rows; k RoPE'd and v stored into
//                          the caches at each row's position
//   fk_prefill_attend      causal attention of each row over its sequence's
//                          cache, on the matrix cores, into f16 in the tile
//                          layout (the output projection's A)
//
// Semantics follow src/FuryKernel/Program/Eval.hs (RmsNorm :292-305, Rope
// :634-645, KvStore :331-349, Attend :351-380, Gather :382-392) per row; the
// f16 roundings of the GEMM operands are this target's (the f16 bar).
#pragma once

#include "fk_common.h"
#include "fk_layout.h"
#include "fk_gemm.h"
#include "fk_step.h"  // rope_elem, narrow_cache: the decode step's RoPE and cache rounding

namespace fk {

// binary32 -> binary16, to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t to_f16(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

}  // namespace fk

// x[r] = table[tokens[r]] · factor.  One wave a row, 4 columns a lane at a
// time; rows × width f32 out.  A token past the table reads its last row
// (the host refuses such tokens before they get here).
struct fk_prefill_gather_params {
  uint32_t rows;
  uint32_t width;       // a multiple of 4
  uint32_t table_rows;
  uint32_t table_f16;   // the table is f16 (else f32)
  float factor;
};

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
struct fk_prefill_norm_params {
  uint32_t rows;      // a multiple of 256
  uint32_t width;     // a multiple of 32
  float eps;
  float factor;
  uint32_t has_gamma;
};

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

// q RoPE'd into f16 rows [rows, heads · d]; k RoPE'd and v into the caches
// ([slots][kv_heads][length][d], f16 or bf16) at (slot, head, position mod
// length).  One threadgroup a row.  The cache stores round as the decode
// step's stores do (narrowF16 / narrowBF16).
struct fk_prefill_rope_params {
  uint32_t rows;
  uint32_t heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t rotated;    // pairs RoPE turns
  uint32_t rope_rows;  // positions the RoPE table holds
  uint32_t length;     // ring length
  uint32_t slots;
  uint32_t cache_bf16;
};

extern "C" __global__ void __launch_bounds__(256) fk_prefill_rope_store(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot, const float *__restrict__ rope,
    uint16_t *__restrict__ qr, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, fk_prefill_rope_params p) {
  const uint32_t row = blockIdx.x;
  const uint32_t d = p.head_dim;
  const uint32_t pos = position[row];
  const uint32_t sl = min(slot[row], p.slots - 1);
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  const uint32_t qw = p.heads * d, kw = p.kv_heads * d;
  const float *qx = q + (size_t)row * qw;
  const float *kx = k + (size_t)row * kw;
  const float *vx = v + (size_t)row * kw;
  const bool bf16 = p.cache_bf16 != 0;
  for (uint32_t e = threadIdx.x; e < qw + 2 * kw; e += blockDim.x) {
    if (e < qw) {
      qr[(size_t)row * qw + e] = fk::to_f16(fk::rope_elem(qx + (e / d) * d, e % d, d, p.rotated, cs));
    } else {
      const uint32_t f = e < qw + kw ? e - qw : e - qw - kw;
      const uint32_t h = f / d, i = f % d;
      const size_t at = (((size_t)sl * p.kv_heads + h) * p.length + pos % p.length) * d + i;
      if (e < qw + kw)
        kc[at] = fk::narrow_cache(fk::rope_elem(kx + h * d, i, d, p.rotated, cs), bf16);
      else
        vc[at] = fk::narrow_cache(vx[f], bf16);
    }
  }
}

// Causal attention of a step's rows over their sequences' caches, on the
// matrix cores.  A threadgroup takes 32 rows (one sequence's, consecutive
// positions p0 .. p0 + 31) and one kv head (grid: rows / 32 × kv_heads,
// query blocks first); its G wavefronts are the G query heads of that kv head.  Keys go by blocks of 32 positions through LDS (K
// rows padded to 144 bytes, V transposed); a wavefront computes Sᵀ = K Qᵀ
// (v_mfma_f32_32x32x16_f16: lane l holds query l mod 32 and 16 of the
// block's keys), the online softmax in binary32 (a query's maximum and sum
// from its two lanes), and Oᵀ += Vᵀ Pᵀ with Pᵀ rounded to f16 straight from
// the scores' registers.  Head dimension 64.  Output: O / sum into the tile
// layout of [rows, heads · 64], the output projection's A.
struct fk_prefill_attend_params {
  uint32_t rows;        // a multiple of 32
  uint32_t heads;
  uint32_t kv_heads;    // heads / kv_heads (G) is 1, 2 or 4
  uint32_t length;      // ring length
  uint32_t slots;
  uint32_t window;      // 0: none; else a row sees positions > position - window
  uint32_t cache_bf16;
  float scale;
};

#define FK_ATT_KROW 72   // halves a staged K row takes: 64 and 8 of padding
#define FK_ATT_VROW 40   // halves a staged Vᵀ row (one d, 32 keys) takes: 32 and 8 of padding

extern "C" __global__ void __launch_bounds__(256) fk_prefill_attend(
    const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot, uint16_t *__restrict__ out,
    fk_prefill_attend_params p) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[32 * FK_ATT_KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vts[64 * FK_ATT_VROW];
  const uint32_t G = p.heads / p.kv_heads;
  const uint32_t nthreads = G * FK_WAVE;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  const uint32_t qblocks = p.rows / 32;
  const uint32_t r0 = (blockIdx.x % qblocks) * 32;   // the block's first row
  const uint32_t g = blockIdx.x / qblocks;           // kv head
  const uint32_t h = g * G + wave;                   // this wavefront's query head
  const uint32_t p0 = position[r0];
  const uint32_t sl = min(slot[r0], p.slots - 1);
  const bool bf16 = p.cache_bf16 != 0;
  const uint32_t qw = p.heads * 64;
  const uint32_t qrow = r0 + lane % 32;
  const uint32_t qpos = p0 + lane % 32;              // this lane's query position

  // Qᵀ fragments (B of Sᵀ = K Qᵀ): lane l holds Q[query l mod 32][16 c + 8 (l div 32) .. + 7].
  fk::Half8 qf[4];
#pragma unroll
  for (int c = 0; c < 4; c++)
    qf[c].u = *reinterpret_cast<const uint4 *>(qr + (size_t)qrow * qw + h * 64 + 16 * c + 8 * (lane / 32));

  fk_float16v o[2];   // Oᵀ: d-block db, lane l's query l mod 32, d = 32 db + 8 gg + 4 (l div 32) + r
#pragma unroll
  for (int r = 0; r < 16; r++) {
    o[0][r] = 0.0f;
    o[1][r] = 0.0f;
  }
  float mrun = -__builtin_inff(), lrun = 0.0f;

  const uint32_t last_pos = p0 + 31;
  const uint32_t first_pos = p.window && p0 + 1 > p.window ? p0 + 1 - p.window : 0;
  const size_t cache_base = ((size_t)sl * p.kv_heads + g) * p.length * 64;
  for (uint32_t kb = first_pos / 32; kb * 32 <= last_pos; kb++) {
    // Stage the block's K rows and Vᵀ: 32 keys × 64 d each, 16 bytes a
    // thread at a time; keys past the block's last query stay zero.
    __syncthreads();
    for (uint32_t u = tid; u < 32 * 8; u += nthreads) {
      const uint32_t key = u / 8, c8 = (u % 8) * 8;
      const uint32_t kp = kb * 32 + key;
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (kp <= last_pos) {
        const size_t at = cache_base + (size_t)(kp % p.length) * 64 + c8;
        kv = *reinterpret_cast<const uint4 *>(kc + at);
        vv = *reinterpret_cast<const uint4 *>(vc + at);
      }
      if (bf16) {  // the matrix operations take f16: widen bf16, narrow to f16
        uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          kw[e] = fk::to_f16(__uint_as_float(kw[e] << 16)) | ((uint32_t)fk::to_f16(__uint_as_float(kw[e] & 0xffff0000u)) << 16);
          vw[e] = fk::to_f16(__uint_as_float(vw[e] << 16)) | ((uint32_t)fk::to_f16(__uint_as_float(vw[e] & 0xffff0000u)) << 16);
        }
        kv = make_uint4(kw[0], kw[1], kw[2], kw[3]);
        vv = make_uint4(vw[0], vw[1], vw[2], vw[3]);
      }
      *reinterpret_cast<uint4 *>(ks + key * FK_ATT_KROW + c8) = kv;
      const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        vts[(c8 + 2 * e) * FK_ATT_VROW + key] = (uint16_t)(vw[e] & 0xffffu);
        vts[(c8 + 2 * e + 1) * FK_ATT_VROW + key] = (uint16_t)(vw[e] >> 16);
      }
    }
    __syncthreads();

    // Sᵀ = K Qᵀ: 4 chunks of 16 d.  A = K: lane l holds K[key l mod 32][16 c + 8 (l div 32) .. + 7].
    fk_float16v s;
#pragma unroll
    for (int r = 0; r < 16; r++) s[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      fk::Half8 kf;
      kf.u = *reinterpret_cast<const uint4 *>(ks + (lane % 32) * FK_ATT_KROW + 16 * c + 8 * (lane / 32));
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf.h, qf[c].h, s, 0, 0, 0);
    }
    // Register 4 gg + r: key kb 32 + 8 gg + 4 (l div 32) + r of query qpos.
    float mblk = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t kp = kb * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
      const bool ok = kp <= qpos && kp >= (p.window && qpos + 1 > p.window ? qpos + 1 - p.window : 0u);
      s[r] = ok ? s[r] * p.scale : -__builtin_inff();
      mblk = fmaxf(mblk, s[r]);
    }
    mblk = fmaxf(mblk, __shfl_xor(mblk, 32));
    const float mnew = fmaxf(mrun, mblk);
    // A row that has seen no key yet keeps nothing (its maximum is -inf).
    const float alpha = mnew == -__builtin_inff() ? 1.0f : __expf(mrun - mnew);
    float psum = 0.0f;
    fk::Half8 pf[2];   // Pᵀ chunks (B of Oᵀ += Vᵀ Pᵀ): registers 8 c .. 8 c + 7
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float e = mnew == -__builtin_inff() ? 0.0f : __expf(s[r] - mnew);
      psum += e;
      pf[r / 8].h[r % 8] = (_Float16)e;
    }
    psum += __shfl_xor(psum, 32);
    lrun = lrun * alpha + psum;
    mrun = mnew;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      o[0][r] *= alpha;
      o[1][r] *= alpha;
    }
    // Oᵀ += Vᵀ Pᵀ.  Chunk c's k index 8 (l div 32) + e is key 16 c + 8 (e div 4)
    // + 4 (l div 32) + e mod 4 (the scores' register order); A = Vᵀ: lane l
    // holds V[those keys][d = 32 db + l mod 32], two runs of 4 keys.
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const uint16_t *vrow = vts + (32 * db + lane % 32) * FK_ATT_VROW + 16 * c + 4 * (lane / 32);
        const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
        const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 8);
        fk::Half8 vf;
        vf.u = make_uint4(lo.x, lo.y, hi.x, hi.y);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf.h, pf[c].h, o[db], 0, 0, 0);
      }
  }

  // O = Oᵀ / sum into the tile layout: lane l's query row, d = 32 db + 8 gg +
  // 4 (l div 32) .. + 3, four consecutive columns a store.
  const float inv = 1.0f / lrun;
#pragma unroll
  for (int db = 0; db < 2; db++)
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
      const uint32_t col = h * 64 + 32 * db + 8 * gg + 4 * (lane / 32);
      const uint32_t lo = fk::to_f16(o[db][4 * gg] * inv) | ((uint32_t)fk::to_f16(o[db][4 * gg + 1] * inv) << 16);
      const uint32_t hi = fk::to_f16(o[db][4 * gg + 2] * inv) | ((uint32_t)fk::to_f16(o[db][4 * gg + 3] * inv) << 16);
      *reinterpret_cast<uint2 *>(out + fk::tile_offset(qrow, col, qw)) = make_uint2(lo, hi);
    }
}

// The greedy token of each row: the index of its largest logit, the first
// of equals, by the decode step's 64-bit keys (value order, then the
// complement of the index; a NaN at index 0 wins, elsewhere loses:
// src/FuryKernel/Program/Eval.hs:681-685).  One wave a row.
struct fk_prefill_argmax_params {
  uint32_t rows;
  uint32_t width;
};

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
