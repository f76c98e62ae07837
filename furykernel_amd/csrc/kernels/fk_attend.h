// fk_attend.h — the prefill's causal attention on the matrix cores
// (src/FuryKernel/Program/Eval.hs:351-380 per row).  Built into a code object
// of its own (fk_attend.hip) with the compiler's VGPR form of the matrix
// operations: the online softmax rescales its output accumulators with
// plain arithmetic, which on accumulators held in AGPRs would copy them out
// and back every block of keys.
#pragma once

#include "fk_common.h"
#include "fk_layout.h"
#include "fk_mfma.h"

// Causal attention of a step's rows over their sequences' caches, on the
// matrix cores.  A threadgroup takes 32 rows (one sequence's, consecutive
// positions p0 .. p0 + 31) and one kv head (grid: rows / 32 × kv_heads,
// query blocks first); its G wavefronts are the G query heads of that kv
// head.  Keys go by blocks of 32 positions through LDS (K rows padded to 144
// bytes, V transposed); a wavefront computes Sᵀ = K Qᵀ
// (v_mfma_f32_32x32x16_f16: lane l holds query l mod 32 and 16 of the
// block's keys), the online softmax in binary32 — exp2 of one FMA of the
// score, the scale·log2 e and the running maximum; the causal and window
// masks only on the blocks that cross them; the output rescaled only when a
// maximum moved — and Oᵀ += Vᵀ Pᵀ with Pᵀ rounded to f16 straight from the
// scores' registers.  Head dimension 64.  Output: O / sum into the tile
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
#define FK_ATT_VROW 34   // halves a staged Vᵀ row (one d, 32 keys) takes: 32 and 2, so that rows 17 banks
                         // apart keep both the staging writes and the fragment reads on distinct banks

namespace fk {

// bf16 pairs of a word -> f16 pairs (the matrix operations take f16).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  return to_f16(__uint_as_float(w << 16)) | ((uint32_t)to_f16(__uint_as_float(w & 0xffff0000u)) << 16);
}

}  // namespace fk

template <uint32_t G>
__device__ __forceinline__ void prefill_attend(const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc,
                                               const uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                                               const uint32_t *__restrict__ slot, uint16_t *__restrict__ out,
                                               const fk_prefill_attend_params &p) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[32 * FK_ATT_KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vts[64 * FK_ATT_VROW];
  constexpr uint32_t nthreads = G * FK_WAVE;
  constexpr uint32_t per = 256 / nthreads;   // staging units a thread
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
  const uint32_t qfirst = p.window && qpos + 1 > p.window ? qpos + 1 - p.window : 0u;
  const float c = p.scale * 1.4426950408889634f;      // scores to log2 units

  // Qᵀ fragments (B of Sᵀ = K Qᵀ): lane l holds Q[query l mod 32][16 c + 8 (l div 32) .. + 7].
  fk::Half8 qf[4];
#pragma unroll
  for (int k4 = 0; k4 < 4; k4++)
    qf[k4].u = *reinterpret_cast<const uint4 *>(qr + (size_t)qrow * qw + h * 64 + 16 * k4 + 8 * (lane / 32));

  fk_float16v o[2];   // Oᵀ: d-block db, lane l's query, d = 32 db + 8 gg + 4 (l div 32) + r
#pragma unroll
  for (int r = 0; r < 16; r++) {
    o[0][r] = 0.0f;
    o[1][r] = 0.0f;
  }
  float mrun = -__builtin_inff(), lrun = 0.0f;

  const uint32_t last_pos = p0 + 31;
  const uint32_t first_pos = p.window && p0 + 1 > p.window ? p0 + 1 - p.window : 0;
  // Blocks with every key visible to every row of the block need no mask.
  const uint32_t win_lo = p.window && last_pos + 1 > p.window ? last_pos + 1 - p.window : 0;
  const size_t cache_base = ((size_t)sl * p.kv_heads + g) * p.length * 64;
  for (uint32_t kb = first_pos / 32; kb * 32 <= last_pos; kb++) {
    // The block's first key in the ring (a ring length is a multiple of 32,
    // so the block does not wrap).
    const uint32_t ring0 = (kb * 32) % p.length;
    // Stage the block's K rows (unit u: key u div 8, d 8 (u mod 8) .. + 7,
    // 16 bytes) and Vᵀ (item u: keys 2 (u div 16) and the next, d 4 (u mod
    // 16) .. + 3: four dwords of two keys each); keys past the block's last
    // query stay zero.
    __syncthreads();
#pragma unroll
    for (uint32_t e = 0; e < per; e++) {
      const uint32_t u = tid + e * nthreads;
      const uint32_t key = u / 8, c8 = (u % 8) * 8;
      uint4 kv = make_uint4(0, 0, 0, 0);
      if (kb * 32 + key <= last_pos) kv = *reinterpret_cast<const uint4 *>(kc + cache_base + (size_t)(ring0 + key) * 64 + c8);
      if (bf16)
        kv = make_uint4(fk::bf16x2_to_f16x2(kv.x), fk::bf16x2_to_f16x2(kv.y), fk::bf16x2_to_f16x2(kv.z),
                        fk::bf16x2_to_f16x2(kv.w));
      *reinterpret_cast<uint4 *>(ks + key * FK_ATT_KROW + c8) = kv;
      const uint32_t k2 = 2 * (u / 16), d4 = 4 * (u % 16);
      uint2 va = make_uint2(0, 0), vb = make_uint2(0, 0);
      if (kb * 32 + k2 <= last_pos) va = *reinterpret_cast<const uint2 *>(vc + cache_base + (size_t)(ring0 + k2) * 64 + d4);
      if (kb * 32 + k2 + 1 <= last_pos)
        vb = *reinterpret_cast<const uint2 *>(vc + cache_base + (size_t)(ring0 + k2 + 1) * 64 + d4);
      if (bf16) {
        va = make_uint2(fk::bf16x2_to_f16x2(va.x), fk::bf16x2_to_f16x2(va.y));
        vb = make_uint2(fk::bf16x2_to_f16x2(vb.x), fk::bf16x2_to_f16x2(vb.y));
      }
      uint32_t *vt = reinterpret_cast<uint32_t *>(vts);
      vt[((d4 + 0) * FK_ATT_VROW + k2) / 2] = (va.x & 0xffffu) | (vb.x << 16);
      vt[((d4 + 1) * FK_ATT_VROW + k2) / 2] = (va.x >> 16) | (vb.x & 0xffff0000u);
      vt[((d4 + 2) * FK_ATT_VROW + k2) / 2] = (va.y & 0xffffu) | (vb.y << 16);
      vt[((d4 + 3) * FK_ATT_VROW + k2) / 2] = (va.y >> 16) | (vb.y & 0xffff0000u);
    }
    __syncthreads();

    // Sᵀ = K Qᵀ: 4 chunks of 16 d.  A = K: lane l holds K[key l mod 32][16 c + 8 (l div 32) .. + 7].
    fk_float16v s;
#pragma unroll
    for (int r = 0; r < 16; r++) s[r] = 0.0f;
#pragma unroll
    for (int k4 = 0; k4 < 4; k4++) {
      fk::Half8 kf;
      kf.u = *reinterpret_cast<const uint4 *>(ks + (lane % 32) * FK_ATT_KROW + 16 * k4 + 8 * (lane / 32));
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf.h, qf[k4].h, s, 0, 0, 0);
    }
    // Register 4 gg + r: key kb 32 + 8 gg + 4 (l div 32) + r of query qpos.
    // The mask where the block crosses the causal edge or the window's start.
    if (kb * 32 + 31 > p0 || kb * 32 < win_lo) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const uint32_t kp = kb * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
        s[r] = kp <= qpos && kp >= qfirst ? s[r] : -__builtin_inff();
      }
    }
    float mblk = s[0];
#pragma unroll
    for (int r = 1; r < 16; r++) mblk = fmaxf(mblk, s[r]);
    mblk = fmaxf(mblk, __shfl_xor(mblk, 32));
    const float mnew = fmaxf(mrun, mblk);
    // A row that has seen no key yet keeps nothing (its maximum is -inf).
    const bool none = mnew == -__builtin_inff();
    const float mc = none ? 0.0f : mnew * c;
    float psum = 0.0f;
    fk::Half8 pf[2];   // Pᵀ chunks (B of Oᵀ += Vᵀ Pᵀ): registers 8 k2 .. 8 k2 + 7
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float e = none ? 0.0f : __builtin_amdgcn_exp2f(fmaf(s[r], c, -mc));
      psum += e;
      pf[r / 8].h[r % 8] = (_Float16)e;
    }
    psum += __shfl_xor(psum, 32);
    // Rescale what the rows have so far only when some maximum moved.
    if (__any(mnew != mrun)) {
      const float alpha = none || mrun == -__builtin_inff() ? (none ? 1.0f : 0.0f)
                                                            : __builtin_amdgcn_exp2f(mrun * c - mc);
      lrun *= alpha;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        o[0][r] *= alpha;
        o[1][r] *= alpha;
      }
    }
    lrun += psum;
    mrun = mnew;
    // Oᵀ += Vᵀ Pᵀ.  Chunk k2's k index 8 (l div 32) + e is key 16 k2 + 8 (e div 4)
    // + 4 (l div 32) + e mod 4 (the scores' register order); A = Vᵀ: lane l
    // holds V[those keys][d = 32 db + l mod 32], two runs of 4 keys.
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int k2 = 0; k2 < 2; k2++) {
        const uint32_t *vrow = reinterpret_cast<const uint32_t *>(vts) +
                               ((32 * db + lane % 32) * FK_ATT_VROW + 16 * k2 + 4 * (lane / 32)) / 2;
        fk::Half8 vf;
        vf.u = make_uint4(vrow[0], vrow[1], vrow[4], vrow[5]);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf.h, pf[k2].h, o[db], 0, 0, 0);
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

// One entry a group size G = heads / kv_heads (threads 64 G).
#define FK_PREFILL_ATTEND(G)                                                                                    \
  extern "C" __global__ void __launch_bounds__(64 * G) fk_prefill_attend_g##G(                                  \
      const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,       \
      const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot, uint16_t *__restrict__ out,   \
      fk_prefill_attend_params p) {                                                                             \
    prefill_attend<G>(qr, kc, vc, position, slot, out, p);                                                      \
  }
FK_PREFILL_ATTEND(1)
FK_PREFILL_ATTEND(2)
FK_PREFILL_ATTEND(4)

