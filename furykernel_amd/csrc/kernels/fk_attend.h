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

#define FK_ATT_LDS __attribute__((address_space(3)))

// Causal attention of a step's rows over their sequences' caches, on the
// matrix cores.  A threadgroup takes 32 rows (one sequence's, consecutive
// positions p0 .. p0 + 31) and one kv head (grid: rows / 32 × kv_heads,
// query blocks first); its G wavefronts are the G query heads of that kv
// head.  Keys go by blocks of 64 positions through two LDS buffers: while a
// block is multiplied, the next block's K and V rows are on their way from
// the caches into registers, and go into the other buffer after; one
// barrier a block.  A wavefront computes Sᵀ = K Qᵀ
// (v_mfma_f32_32x32x16_f16: lane l holds query l mod 32 and 16 keys of each
// half block), the online softmax in binary32 — exp2 of one FMA of the
// score, the scale·log2 e and the running maximum; the causal and window
// masks only on the blocks that cross them; the output rescaled only when a
// maximum moved; the row sums from the f16 probabilities the matrix
// operation takes (v_dot2) — and Oᵀ += Vᵀ Pᵀ with Pᵀ rounded to f16 straight
// from the scores' registers and Vᵀ read transposed out of V's rows
// (ds_read_b64_tr_b16).  Head dimension 64.  Output: O / sum into the tile
// layout of [rows, heads · 64], the output projection's A.

#define FK_ATT_KB 64     // keys a block
#define FK_ATT_TABLE 256 // a block table's entries the direct paged form holds in LDS
// Staged rows are 64 halves (128 bytes), swizzled rather than padded.  K: a
// row's 16-byte unit u sits at u ^ ((key >> 1) mod 8), so that the fragment
// reads (16 lanes: 16 keys, one unit) meet 16 different bank groups and the
// staging writes (16 lanes: 2 keys' 8 units) too.  V: the two 64-byte halves
// of a row swap places when key bit 1 is set, so that a transposed read's 4
// consecutive rows × 64 bytes cover the 256 bytes of banks once.
__device__ __forceinline__ uint32_t fk_att_kplace(uint32_t key, uint32_t half_off) {
  return key * 64 + (half_off ^ (((key >> 1) & 7u) << 3));
}
__device__ __forceinline__ uint32_t fk_att_vplace(uint32_t key, uint32_t half_off) {
  return key * 64 + (half_off ^ (((key >> 1) & 1u) << 5));
}

namespace fk {

// bf16 pairs of a word -> f16 pairs (the matrix operations take f16).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  return to_f16(__uint_as_float(w << 16)) | ((uint32_t)to_f16(__uint_as_float(w & 0xffff0000u)) << 16);
}

__device__ __forceinline__ uint4 bf16x8_to_f16x8(uint4 v) {
  return make_uint4(bf16x2_to_f16x2(v.x), bf16x2_to_f16x2(v.y), bf16x2_to_f16x2(v.z), bf16x2_to_f16x2(v.w));
}

}  // namespace fk

typedef short fk_short4 __attribute__((ext_vector_type(4)));
typedef _Float16 fk_half2 __attribute__((ext_vector_type(2)));
typedef float fk_float2v __attribute__((ext_vector_type(2)));

// PG: the caches are paged pools ([blocks][kv_heads][block_size][64]) and
// `slot` the rows' block tables ([rows][table_len]); a block of rows reads
// its first row's table (its rows are one sequence's).
// DIRECT: f16 rings and no staged rows; each block's K and V rows go
// straight from the ring into LDS (direct loads, no registers between), a
// row's units placed by the loads' source addresses as the staging writes
// would place them; keys past the block's last query read that query's own
// row (its score is masked and its probability 0, so a finite row is all
// it needs).
template <uint32_t G, bool PG = false, bool DIRECT = false>
__device__ __forceinline__ void prefill_attend(const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc,
                                               const uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                                               const uint32_t *__restrict__ slot, uint16_t *__restrict__ out,
                                               const uint16_t *__restrict__ kst, const uint16_t *__restrict__ vst,
                                               const fk_prefill_attend_params &p,
                                               const fk_paging &pg = fk_paging{}) {
  // The two buffers of K and of V: four objects (see the direct loop for why).
  __shared__ __attribute__((aligned(16))) uint16_t ks0[FK_ATT_KB * 64], ks1[FK_ATT_KB * 64];
  __shared__ __attribute__((aligned(16))) uint16_t vs0[FK_ATT_KB * 64], vs1[FK_ATT_KB * 64];
  constexpr uint32_t nthreads = G * FK_WAVE;
  constexpr uint32_t per = FK_ATT_KB * 8 / nthreads;   // 16-byte units of K (and of V) a thread stages
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  // Heaviest first: a block's keys grow with its place in its run (a
  // sequence's consecutive positions), so threadgroup j takes, of every run
  // and kv head, the run's last block first, then the one before: the
  // longest blocks start first and the short ones fill in at the end.
  const uint32_t qblocks = p.rows / 32;
  const uint32_t per_run = (p.run_rows ? p.run_rows : p.rows) / 32;  // blocks a run
  const uint32_t runs = qblocks / per_run;
  const uint32_t t_rank = blockIdx.x / (runs * p.kv_heads);
  const uint32_t rest = blockIdx.x % (runs * p.kv_heads);
  const uint32_t r0 = ((rest / p.kv_heads) * per_run + (per_run - 1 - t_rank)) * 32;  // the block's first row
  const uint32_t g = rest % p.kv_heads;                                               // kv head
  const uint32_t h = g * G + wave;                   // this wavefront's query head
  const uint32_t p0 = position[r0];
  const uint32_t sl = PG ? 0u : min(slot[r0], p.slots - 1);
  const uint32_t *const tab = slot + (size_t)r0 * pg.table_len;  // PG: the block's table
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
  // Staged stores (Plan.hs:41-50): the step's own rows of this sequence are
  // not in the ring yet.  Its run of rows starts at row rf (runs of run_rows
  // rows, consecutive positions of one slot), position start; keys from
  // there on are read from the staging rows [rows][kv_heads][64], the
  // earlier ones from the ring.
  const bool staged = !PG && p.staged != 0;
  const uint32_t rf = staged ? (r0 / p.run_rows) * p.run_rows : 0u;
  const uint32_t start = staged ? position[rf] : 0xFFFFFFFFu;

  // Where lane l's transposed V reads start (see softmax_pv).
  const uint32_t tq = lane & 15;
  const uint32_t tr_key = 4 * (lane / 32) + tq / 4;
  const uint32_t tr_d = 16 * ((lane / 16) & 1) + 4 * (tq & 3);

  // A block's K (or V) rows into registers (unit u: key u div 8, d 8 (u mod
  // 8) .. + 7, 16 bytes), keys past the block's last query zero (the ring
  // length is a multiple of 64, so a block does not wrap); then into an LDS
  // buffer, bf16 caches converted on the way (a uniform branch, so that f16
  // caches pay nothing for it).
  uint4 kreg[per], vreg[per];
  // PG: where each of the thread's units of block kb lies in a pool (the
  // keys' and the values' pools alike), looked up once for both.
  size_t poff[per];
  auto locate = [&](uint32_t kb) {
#pragma unroll
    for (uint32_t e = 0; e < per; e++) {
      const uint32_t u = tid + e * nthreads;
      const uint32_t t = kb * FK_ATT_KB + u / 8;
      // position t's block through the table, both clamped into place
      const uint32_t blk = min(tab[min(t / pg.block_size, pg.table_len - 1)], pg.blocks - 1);
      poff[e] = (((size_t)blk * p.kv_heads + g) * pg.block_size + t % pg.block_size) * 64 + (u % 8) * 8;
    }
  };
  auto fetch = [&](uint4 (&reg)[per], const uint16_t *__restrict__ cache, const uint16_t *__restrict__ stage,
                   uint32_t kb) {
    const uint32_t ring0 = (kb * FK_ATT_KB) % p.length;
#pragma unroll
    for (uint32_t e = 0; e < per; e++) {
      const uint32_t u = tid + e * nthreads;
      const uint32_t key = u / 8, c8 = (u % 8) * 8;
      const uint32_t t = kb * FK_ATT_KB + key;
      const bool live = t <= last_pos;
      // A staged row's index, clamped into the step's rows.
      const uint32_t srow = min(rf + (t - min(t, start)), p.rows - 1);
      const uint16_t *src;
      if constexpr (PG) {
        src = cache + poff[e];
      } else {
        src = staged && t >= start ? stage + ((size_t)srow * p.kv_heads + g) * 64 + c8
                                   : cache + cache_base + (size_t)(ring0 + key) * 64 + c8;
      }
      reg[e] = live ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash_k = [&](uint32_t buf) {
    if (bf16) {
#pragma unroll
      for (uint32_t e = 0; e < per; e++) kreg[e] = fk::bf16x8_to_f16x8(kreg[e]);
    }
#pragma unroll
    for (uint32_t e = 0; e < per; e++) {
      const uint32_t u = tid + e * nthreads;
      *reinterpret_cast<uint4 *>(&(buf ? ks1 : ks0)[fk_att_kplace(u / 8, (u % 8) * 8)]) = kreg[e];
    }
  };
  auto stash_v = [&](uint32_t buf) {
    if (bf16) {
#pragma unroll
      for (uint32_t e = 0; e < per; e++) vreg[e] = fk::bf16x8_to_f16x8(vreg[e]);
    }
#pragma unroll
    for (uint32_t e = 0; e < per; e++) {
      const uint32_t u = tid + e * nthreads;
      *reinterpret_cast<uint4 *>(&(buf ? vs1 : vs0)[fk_att_vplace(u / 8, (u % 8) * 8)]) = vreg[e];
    }
  };

  // A block: its scores, the online softmax and Oᵀ += Vᵀ Pᵀ, from K and V
  // buffer buf.  mref is each row's reference maximum in log2 units (score ·
  // scale · log2 e): it moves only when a block's maximum passes it by more
  // than 8, so that Oᵀ and the sum are rescaled rarely; the probabilities
  // exp2(score · c - mref) are then at most 2^8, which f16 holds with its
  // full relative precision, and O / sum does not depend on the reference.
  // A row that has seen no key yet keeps nothing: its reference and every
  // score are -inf, and with mc = 0 each exp2 is exp2(-inf) = 0.
  auto step = [&](uint32_t kb, const uint16_t *kbuf, const uint16_t *vbuf) {
    // Sᵀ = K Qᵀ: two halves of 32 keys, 4 chunks of 16 d each.  A = K: lane
    // l holds K[key 32 sb + l mod 32][16 c + 8 (l div 32) .. + 7].
    fk_float16v sc[2];
#pragma unroll
    for (int sb = 0; sb < 2; sb++) {
#pragma unroll
      for (int r = 0; r < 16; r++) sc[sb][r] = 0.0f;
#pragma unroll
      for (int k4 = 0; k4 < 4; k4++) {
        fk::Half8 kf;
        kf.u = *reinterpret_cast<const uint4 *>(&kbuf[fk_att_kplace(32 * sb + lane % 32, 16 * k4 + 8 * (lane / 32))]);
        sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf.h, qf[k4].h, sc[sb], 0, 0, 0);
      }
    }
    // Register 4 gg + r of half sb: key 32 sb + 8 gg + 4 (l div 32) + r of
    // the block, of query qpos.  The mask where the block crosses the causal
    // edge or the window's start.
    if (kb * FK_ATT_KB + FK_ATT_KB - 1 > p0 || kb * FK_ATT_KB < win_lo) {
#pragma unroll
      for (int sb = 0; sb < 2; sb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const uint32_t kp = kb * FK_ATT_KB + 32 * sb + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
          sc[sb][r] = kp <= qpos && kp >= qfirst ? sc[sb][r] : -__builtin_inff();
        }
    }
    // The block's maximum of each row: three-way maxima down the 32 scores.
    float mblk = __builtin_fmaxf(__builtin_fmaxf(sc[0][0], sc[1][0]), sc[0][1]);
#pragma unroll
    for (int r = 1; r < 16; r++)
      mblk = __builtin_fmaxf(__builtin_fmaxf(mblk, sc[1][r]), r + 1 < 16 ? sc[0][r + 1] : sc[1][r]);
    // The two halves of the wavefront hold the other 32 keys of each query:
    // v_permlane32_swap gives each lane the other half's value (an exchange
    // in the vector ALU, where a shuffle would go through LDS).
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mblk), __float_as_uint(mblk), false, false);
      mblk = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;
    }
    const bool passed = mblk > mrun + 8.0f;
    if (__any(passed)) {
      const float mnew = passed ? mblk : mrun;
      const float alpha = mnew == mrun ? 1.0f : __builtin_amdgcn_exp2f(mrun - mnew);
      lrun *= alpha;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        o[0][r] *= alpha;
        o[1][r] *= alpha;
      }
      mrun = mnew;
    }
    const float mc = mrun == -__builtin_inff() ? 0.0f : mrun;

    // Pᵀ chunk 2 sb + k2 (B of Oᵀ += Vᵀ Pᵀ): registers 8 k2 .. 8 k2 + 7 of
    // half sb, converted in pairs; the row's sum taken from those same f16
    // pairs, as the matrix operation takes them.
    fk::Half8 pf[4];
    float psum = 0.0f;
    const fk_half2 ones = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int sb = 0; sb < 2; sb++)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float e0 = __builtin_amdgcn_exp2f(fmaf(sc[sb][r], c, -mc));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(sc[sb][r + 1], c, -mc));
        const fk_half2 pair = __builtin_convertvector((fk_float2v){e0, e1}, fk_half2);
        reinterpret_cast<fk_half2 *>(&pf[2 * sb + r / 8])[(r % 8) / 2] = pair;
        psum = __builtin_amdgcn_fdot2(pair, ones, psum, false);
      }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(psum), __float_as_uint(psum), false, false);
      lrun += __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    // Oᵀ += Vᵀ Pᵀ, chunk by chunk.  Transposed V reads: within each 16
    // lanes, lane 4 k + q reads key K0 + k, d D0 + 4 q .. + 3 and receives
    // keys K0 .. K0 + 3 of d D0 + (its index in the 16); for chunk (sb, k2)
    // lane l wants d 32 db + l mod 32 and keys 32 sb + 16 k2 + 8 t + 4 (l div
    // 32) + 0 .. 3 (t = 0, 1): the scores' register order, which Pᵀ keeps.
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t key0 = 32 * (q / 2) + 16 * (q % 2) + tr_key;
        const fk_short4 t0 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((FK_ATT_LDS fk_short4 *)&vbuf[fk_att_vplace(key0, 32 * db + tr_d)]);
        const fk_short4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (FK_ATT_LDS fk_short4 *)&vbuf[fk_att_vplace(key0 + 8, 32 * db + tr_d)]);
        const uint2 w0 = __builtin_bit_cast(uint2, t0), w1 = __builtin_bit_cast(uint2, t1);
        fk::Half8 vf;
        vf.u = make_uint4(w0.x, w0.y, w1.x, w1.y);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf.h, pf[q].h, o[db], 0, 0, 0);
      }
  };

  // The loop: while block kb is multiplied from one pair of LDS buffers,
  // block kb + 1's K and V rows are on their way from the caches into
  // registers, and go into the other pair after (every wavefront left it at
  // the last barrier); one barrier a block.
  const uint32_t kb0 = first_pos / FK_ATT_KB, kb_last = last_pos / FK_ATT_KB;
  if constexpr (DIRECT) {
    // Block kb's rows into buffer buf: wavefront w's q-th load fills keys
    // 8 (w NQ + q) .. + 7 (1 KB), lane L unit L mod 8 of key L div 8's row.
    // A ring's rows are read relative to the (slot, kv head) ring; a pool's
    // relative to the pool (under 4 GiB), through the threadgroup's block
    // table, which goes into LDS first (its blocks clamped into the pool).
    constexpr uint32_t NQ = 8 / G;
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);
    const size_t span = PG ? (size_t)pg.blocks * p.kv_heads * pg.block_size * 128 : (size_t)p.length * 128;
    const auto krs = fk::buffer(PG ? kc : kc + cache_base, span);
    const auto vrs = fk::buffer(PG ? vc : vc + cache_base, span);
    const uint32_t last_row = PG ? 0u : last_pos % p.length;
    __shared__ uint32_t ltab[PG ? FK_ATT_TABLE : 1];
    if constexpr (PG) {
      const uint32_t used = min(last_pos / pg.block_size + 1, pg.table_len);
      for (uint32_t i = tid; i < used; i += nthreads) ltab[i] = min(tab[i], pg.blocks - 1);
      __syncthreads();
    }
    // A ring block whose keys all come before the block's last query reads
    // rows ring0 .. ring0 + 63 as they lie: each load's lane part of the
    // address (the key's row and unit) is the same every block and the
    // block's part a scalar offset, so such blocks spend no vector
    // operations on addresses.
    uint32_t kvo[NQ], vvo[NQ];
#pragma unroll
    for (uint32_t q = 0; q < NQ; q++) {
      const uint32_t key = (wave * NQ + q) * 8 + lane / 8, slot_u = lane % 8;
      kvo[q] = key * 128 + (slot_u ^ ((key >> 1) & 7u)) * 16;
      vvo[q] = key * 128 + (slot_u ^ (((key >> 1) & 1u) << 2)) * 16;
    }
    auto fetch_direct = [&](uint32_t kb, uint16_t *kdst, uint16_t *vdst) {
      const uint32_t ring0 = PG ? 0u : (kb * FK_ATT_KB) % p.length;
      if (!PG && kb * FK_ATT_KB + FK_ATT_KB - 1 <= last_pos) {
        const uint32_t so = ring0 * 128;
#pragma unroll
        for (uint32_t q = 0; q < NQ; q++) {
          const uint32_t at = (wave_s * NQ + q) * 1024;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (FK_ATT_LDS char *)kdst + at, 16, kvo[q], so, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (FK_ATT_LDS char *)vdst + at, 16, vvo[q], so, 0, 0);
        }
        return;
      }
#pragma unroll
      for (uint32_t q = 0; q < NQ; q++) {
        const uint32_t key = (wave * NQ + q) * 8 + lane / 8, slot_u = lane % 8;
        uint32_t row;  // the key's row (of 64 halves) in the ring or the pool
        if constexpr (PG) {
          const uint32_t t = min(kb * FK_ATT_KB + key, last_pos);
          row = (ltab[min(t / pg.block_size, pg.table_len - 1)] * p.kv_heads + g) * pg.block_size + t % pg.block_size;
        } else {
          row = kb * FK_ATT_KB + key <= last_pos ? ring0 + key : last_row;
        }
        const uint32_t ku = slot_u ^ ((key >> 1) & 7u);         // K: unit u at place u ^ ((key >> 1) mod 8)
        const uint32_t vu = slot_u ^ (((key >> 1) & 1u) << 2);  // V: the row's halves swapped when key bit 1 is set
        const uint32_t at = (wave_s * NQ + q) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (FK_ATT_LDS char *)kdst + at, 16, (row * 64 + ku * 8) * 2,
                                                 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (FK_ATT_LDS char *)vdst + at, 16, (row * 64 + vu * 8) * 2,
                                                 0, 0, 0);
      }
    };
    // A block: block kb + 1's loads into one pair of buffers, then block kb
    // multiplied from the other.  The compiler makes a read of LDS wait for
    // every direct load into LDS that it cannot tell apart from the read, so
    // that without the restrict-qualified buffers each block's reads waited
    // for the next block's loads to land, and the loads' latency was paid a
    // block; with them the loads fly during the block.
    auto blk = [&](uint32_t kb, const uint16_t *__restrict__ kbuf, const uint16_t *__restrict__ vbuf,
                   uint16_t *__restrict__ kdst, uint16_t *__restrict__ vdst) {
      if (kb < kb_last) fetch_direct(kb + 1, kdst, vdst);
      step(kb, kbuf, vbuf);
    };
    fetch_direct(kb0, ks0, vs0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (uint32_t kb = kb0; kb <= kb_last; kb++) {
      const bool odd = (kb - kb0) & 1;
      blk(kb, odd ? ks1 : ks0, odd ? vs1 : vs0, odd ? ks0 : ks1, odd ? vs0 : vs1);
      __builtin_amdgcn_s_waitcnt(0);  // this wavefront's loads of block kb + 1 landed
      __syncthreads();
    }
  } else {
  if constexpr (PG) locate(kb0);
  fetch(kreg, kc, kst, kb0);
  fetch(vreg, vc, vst, kb0);
  stash_k(0);
  stash_v(0);
  __syncthreads();
  for (uint32_t kb = kb0; kb <= kb_last; kb++) {
    const uint32_t buf = (kb - kb0) & 1;
    if (kb < kb_last) {
      if constexpr (PG) locate(kb + 1);
      fetch(kreg, kc, kst, kb + 1);
      fetch(vreg, vc, vst, kb + 1);
    }
    step(kb, buf ? ks1 : ks0, buf ? vs1 : vs0);
    if (kb < kb_last) {
      stash_k(buf ^ 1);
      stash_v(buf ^ 1);
    }
    __syncthreads();
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
  extern "C" __global__ void __launch_bounds__(64 * G) fk_prefill_attend_g##G(                         \
      const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,       \
      const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot, uint16_t *__restrict__ out,   \
      const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs, fk_prefill_attend_params p) {          \
    prefill_attend<G>(qr, kc, vc, position, slot, out, ks, vs, p);                                              \
  }
FK_PREFILL_ATTEND(1)
FK_PREFILL_ATTEND(2)
FK_PREFILL_ATTEND(4)

// The same over f16 rings with no staged rows, each block's rows loaded
// straight into LDS (the same bindings; ks and vs unused).
#define FK_PREFILL_ATTEND_F16(G)                                                                                \
  extern "C" __global__ void __launch_bounds__(64 * G) fk_prefill_attend_f16_g##G(                     \
      const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,       \
      const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot, uint16_t *__restrict__ out,   \
      const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs, fk_prefill_attend_params p) {          \
    prefill_attend<G, false, true>(qr, kc, vc, position, slot, out, nullptr, nullptr, p);                      \
  }
FK_PREFILL_ATTEND_F16(1)
FK_PREFILL_ATTEND_F16(2)
FK_PREFILL_ATTEND_F16(4)

// The same over paged pools: kc and vc the pools, `table` the rows' block
// tables; no staged rows.
#define FK_PREFILL_ATTEND_PAGED(G)                                                                                \
  extern "C" __global__ void __launch_bounds__(64 * G) fk_prefill_attend_paged_g##G(                             \
      const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,         \
      const uint32_t *__restrict__ position, const uint32_t *__restrict__ table, uint16_t *__restrict__ out,     \
      fk_prefill_attend_paged_params p) {                                                                        \
    prefill_attend<G, true>(qr, kc, vc, position, table, out, nullptr, nullptr, p.a, p.g);                       \
  }
FK_PREFILL_ATTEND_PAGED(1)
FK_PREFILL_ATTEND_PAGED(2)
FK_PREFILL_ATTEND_PAGED(4)

// The same over f16 pools (under 4 GiB, tables of at most FK_ATT_TABLE
// blocks), each block's rows loaded straight into LDS.
#define FK_PREFILL_ATTEND_PAGED_F16(G)                                                                            \
  extern "C" __global__ void __launch_bounds__(64 * G) fk_prefill_attend_paged_f16_g##G(                         \
      const uint16_t *__restrict__ qr, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,         \
      const uint32_t *__restrict__ position, const uint32_t *__restrict__ table, uint16_t *__restrict__ out,     \
      fk_prefill_attend_paged_params p) {                                                                        \
    prefill_attend<G, true, true>(qr, kc, vc, position, table, out, nullptr, nullptr, p.a, p.g);                 \
  }
FK_PREFILL_ATTEND_PAGED_F16(1)
FK_PREFILL_ATTEND_PAGED_F16(2)
FK_PREFILL_ATTEND_PAGED_F16(4)

