// fk_attention.h — the decode attention over a ring cache and the combine of
// its splits (src/FuryKernel/Program/Eval.hs:474-527, the plan's Partials and
// Combine steps, src/FuryKernel/Program/Plan.hs:174-181), as device functions:
// the planned step's launches (fk_step.h) and the library's one-call attention
// (fk_ops.hip) run the same code.
#pragma once

#include "fk_common.h"

// Attention ----------------------------------------------------------------

#define FK_ATTN_MAX_SPLIT 128
#define FK_ATTN_MAX_GROUP 8
#define FK_ATTN_MAX_DIM 64
#define FK_ATTN_THREADS 512
#define FK_ATTN_WAVES (FK_ATTN_THREADS / FK_WAVE)
// A key row in LDS: 64 halves and 8 of padding (144 bytes), so that lanes
// reading 16 bytes of consecutive rows hit distinct banks.
#define FK_ATTN_KROW (FK_ATTN_MAX_DIM + 8)

namespace fk {

// LDS of one attention threadgroup.
struct AttendLds {
  alignas(16) float qs[FK_ATTN_MAX_GROUP * FK_ATTN_MAX_DIM];
  alignas(16) u32x4 ks[FK_ATTN_MAX_SPLIT * FK_ATTN_KROW / 8];   // later: the runs' weighted values
  alignas(16) u32x4 vs[FK_ATTN_MAX_SPLIT * FK_ATTN_MAX_DIM / 8];
  alignas(16) float wt[FK_ATTN_MAX_SPLIT * FK_ATTN_MAX_GROUP];  // [position][head]
  alignas(16) float pm[FK_ATTN_MAX_GROUP * FK_ATTN_WAVES];     // [head][wave]: the maxima of each wave's positions
  alignas(16) float pl[FK_ATTN_WAVES * FK_ATTN_MAX_GROUP];     // [run][head]: the runs' weight sums
};

// A lane's value and its partner's in the other row of its pair of rows
// (lane l ^ 16) or in the other half of the wavefront (lane l ^ 32),
// exchanged in the vector ALU rather than through LDS: of the two words
// v_permlane16_swap / v_permlane32_swap return, one is the lane's own and
// the other its partner's (which is which depends on the row), so only
// order-free uses (a maximum, the sum of two) take them.
__device__ __forceinline__ uint2 rows_pair(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return make_uint2(r[0], r[1]);
}
__device__ __forceinline__ uint2 halves_pair(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return make_uint2(r[0], r[1]);
}

// Head h's largest of the wavefronts' maxima pm[h][wave] (maximumNumber,
// exact whatever the order), on max_key's integers so that no branch
// separates the reads.
__device__ __forceinline__ float waves_max(const float *pm, uint32_t h) {
  static_assert(FK_ATTN_WAVES == 8, "two 16-byte reads of a head's maxima");
  const float4 a = *reinterpret_cast<const float4 *>(pm + h * FK_ATTN_WAVES);
  const float4 b = *reinterpret_cast<const float4 *>(pm + h * FK_ATTN_WAVES + 4);
  const int k = max(max(max(max_key(a.x), max_key(a.y)), max(max_key(a.z), max_key(a.w))),
                    max(max(max_key(b.x), max_key(b.y)), max(max_key(b.z), max_key(b.w))));
  return from_max_key(k);
}

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
// split, score = ((c0 + c1) + (c2 + c3)) * scale, c_j the fused multiply-add
// chain from +0 over the dimensions of quarter j in order (c = fma(q_i, k_i,
// c)); the head's maximum over the split (exact whatever the order); the
// weights exp(score - max), binary64's rounded once.  Over 8 runs of split/8
// positions: the weights' pairwise sum (((w0 + w1) + (w2 + w3)) + ...), a
// position past those the split holds adding +0, and the weighted values in
// order of position from +0 (acc = fma(w, v_i, acc)); then the runs' sums in
// order from +0.  Stored as
// partials: acc[heads][splits][head_dim], then [heads][splits][max, sum] —
// each (head, split)'s values 16-byte aligned for a consumer's vector loads.
// Where the attention's cached rows live: a ring (kc, vc; `slot` the row's
// slot) or paged pools (the blocks' addresses; `slot` the row's block table).
struct CacheRows {
  uint16_t *kc, *vc;
  const uint64_t *kpool, *vpool;
  fk_paging g;
};

// Row t of kv head g of a paged pool: block table[t / block_size] (the table
// index and the block clamped into the table and the pool).
__device__ __forceinline__ uint16_t *paged_row(const uint64_t *pool, const uint32_t *table, const fk_paging &pg,
                                               uint32_t t, uint32_t g, uint32_t d) {
  const uint32_t ti = min(t / pg.block_size, pg.table_len - 1);
  const uint32_t b = min(table[ti], pg.blocks - 1);
  return reinterpret_cast<uint16_t *>(pool[b]) + ((size_t)g * pg.block_size + t % pg.block_size) * d;
}

// PG: the caches are paged pools.  With a reach (p.has_reach), the positions
// run to max(pos, reach[0]) (Graph.hs:223-247), the window's start still the
// row's own position's.
template <uint32_t G, uint32_t D, uint32_t S, int CB, bool PG = false>
__device__ __forceinline__ void attend_split(AttendLds &sh, const float *__restrict__ q,
                                             const float *__restrict__ knew, const float *__restrict__ vnew,
                                             const CacheRows &cr, const uint32_t *__restrict__ position,
                                             const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                             float *__restrict__ partials, const uint32_t *__restrict__ reach,
                                             const fk_step_attend_params &p) {
  uint16_t *__restrict__ kc = cr.kc;
  uint16_t *__restrict__ vc = cr.vc;
  constexpr uint32_t T = FK_ATTN_THREADS;
  static_assert(T == 4 * FK_ATTN_MAX_SPLIT, "four threads a position of the largest split");
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
  const uint32_t sraw = PG ? 0u : slot[0];
  const uint32_t s = sraw < p.slots ? sraw : 0;
  const bool bf16 = CB >= 0 ? CB != 0 : p.cache_bf16 != 0;
  // Positions [first, top], this split's part of them.
  const uint32_t first = (p.window && pos + 1 > p.window) ? pos + 1 - p.window : 0;
  const uint32_t top = p.has_reach ? max(pos, reach[0]) : pos;
  const uint32_t lo = max(first, t * split);
  const uint32_t hi = min(top + 1, (t + 1) * split);
  const uint32_t n = hi > lo ? hi - lo : 0;
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  // A store needs its row's slot (a ring's) or block (a pool's) to exist.
  const bool held = PG ? (pos / cr.g.block_size < cr.g.table_len &&
                          slot[pos / cr.g.block_size] < cr.g.blocks)
                       : sraw < p.slots;
  const bool stores = p.store && held && lo <= pos && pos < hi;
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
  const uint32_t ring0 = PG ? 0u : lo % p.length;
  // The row the new key and value replace (none unless this split stores).
  const uint32_t srow = stores ? pos - lo : 0xFFFFFFFFu;
  // The split's keys, then its values, 16 bytes a load, non-temporal (a step
  // reads each cached row once): K is staged before the scores, V while they
  // are made.  Every load unconditional, a chunk past the split's rows
  // reading its last chunk (or the ring's row lo) and replaced by zeros.
  const uint16_t *kp2[2], *vp2[2];
  bool live2[2];
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint32_t e = tid + m * T;
    live2[m] = e < chunks;
    const uint32_t ec = min(e, chunks > 0 ? chunks - 1 : 0u);
    if constexpr (PG) {
      // A chunk past the split's rows reads the row of position lo.
      const uint32_t at = lo + ec / per_row;
      kp2[m] = paged_row(cr.kpool, slot, cr.g, at, g, d) + 8 * (ec % per_row);
      vp2[m] = paged_row(cr.vpool, slot, cr.g, at, g, d) + 8 * (ec % per_row);
    } else {
      uint32_t ring = ring0 + ec / per_row;
      ring = ring >= p.length ? ring - p.length : ring;
      const size_t at = (base + ring) * d + 8 * (ec % per_row);
      kp2[m] = kc + at;
      vp2[m] = vc + at;
    }
  }
  u32x4 kr[2], vr[2];
#pragma unroll
  for (int m = 0; m < 2; m++) kr[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kp2[m]));
#pragma unroll
  for (int m = 0; m < 2; m++) vr[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vp2[m]));

  // The query rows, RoPE'd as rope_elem does, and the keys into LDS; rows
  // past the positions the split holds get zeros (their weights are zero and
  // their values then add exact zeros).  The new key row replaces row srow.
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
    const uint32_t r = e / per_row;
    if (e < split * per_row && r != srow)
      sh.ks[r * (FK_ATTN_KROW / 8) + e % per_row] = live2[m] ? kr[m] : u32x4{0u, 0u, 0u, 0u};
  }
  uint16_t vh = 0;
  if (stores && tid < d) {
    const uint32_t j = tid;
    const uint32_t i = j < half ? j : j - half;
    float k = kx;
    if (p.krope && i < p.rotated) k = j < half ? kx * kcs - kp * ksn : kx * kcs + kp * ksn;
    const uint16_t kh = narrow_cache(k, bf16);
    vh = narrow_cache(vx, bf16);
    if constexpr (PG) {
      paged_row(cr.kpool, slot, cr.g, pos, g, d)[j] = kh;
      paged_row(cr.vpool, slot, cr.g, pos, g, d)[j] = vh;
    } else {
      const size_t at = (base + pos % p.length) * d + j;
      kc[at] = kh;
      vc[at] = vh;
    }
    ksh[srow * FK_ATTN_KROW + j] = kh;
  }
  __syncthreads();

  // Scores: thread (r, j) = (tid / 4, tid % 4) takes quarter j of position
  // r's key (read once from LDS, widened once) against every head of the
  // group; the quad's four chains are added by DPP, ((c0 + c1) + (c2 + c3)),
  // so each lane of the quad holds every head's score.  Lane 4p + j then
  // keeps heads j and j + 4, and a wavefront's 16 positions give each head's
  // maximum (rotations within rows of 16 lanes, then across rows) into
  // pm[head][wave].
  const uint32_t r = tid / 4;
  const uint32_t jq = tid % 4;
  const uint32_t dq = d / 4;
  constexpr uint32_t HL = FK_ATTN_MAX_GROUP / 4;  // heads a lane keeps
  float hs[HL];
  {
    constexpr uint32_t DQ = FK_ATTN_MAX_DIM / 4;
    const bool live = r < n;
    const uint32_t *krow = reinterpret_cast<const uint32_t *>(sh.ks) + (size_t)min(r, split - 1) * (FK_ATTN_KROW / 2) +
                           jq * (dq / 2);
    float kf[DQ];
#pragma unroll
    for (uint32_t w2 = 0; w2 < DQ / 2; w2++) {
      uint32_t kk = 0u;
      if (w2 < dq / 2) kk = krow[w2];
      kf[2 * w2] = widen_cache((uint16_t)(kk & 0xFFFFu), bf16);
      kf[2 * w2 + 1] = widen_cache((uint16_t)(kk >> 16), bf16);
    }
    float sc[FK_ATTN_MAX_GROUP];
#pragma unroll
    for (uint32_t h = 0; h < FK_ATTN_MAX_GROUP; h++) {
      float c = 0.0f;
      if (h < group) {
        const float *qh = sh.qs + h * d + jq * dq;
#pragma unroll
        for (uint32_t i = 0; i < DQ; i++)
          if (i < dq) c = __builtin_fmaf(qh[i], kf[i], c);
      }
      c = c + dpp_f<0xB1>(c);  // quad_perm [1, 0, 3, 2]: c0 + c1, c2 + c3
      c = c + dpp_f<0x4E>(c);  // quad_perm [2, 3, 0, 1]: (c0 + c1) + (c2 + c3)
      sc[h] = live ? c * p.scale : -__builtin_inff();
    }
#pragma unroll
    for (uint32_t a = 0; a < HL; a++) {
      float v = sc[a * 4];
#pragma unroll
      for (uint32_t q = 1; q < 4; q++) v = jq == q ? sc[a * 4 + q] : v;
      hs[a] = v;
      if (a * 4 < group) {
        int k = max_key(v);
        k = max(k, dpp_i<0x124>(k));  // row_ror:4, the next position of this head
        k = max(k, dpp_i<0x128>(k));  // row_ror:8
        uint2 o = rows_pair((uint32_t)k);
        k = max((int)o.x, (int)o.y);
        o = halves_pair((uint32_t)k);
        k = max((int)o.x, (int)o.y);
        if (lane < 4 && a * 4 + lane < group) sh.pm[(a * 4 + lane) * FK_ATTN_WAVES + wave] = from_max_key(k);
      }
    }
  }
  __syncthreads();
  // The weights exp(score - max), the head's maximum the largest of the
  // wavefronts': thread (r, j) makes heads j and j + 4 (zero past the
  // positions the split holds), then each run's pairwise sum over its
  // positions: at level m (1, 2, 4, 8) lane 4p + j adds the level's sum of
  // position p + m (same head), by row rotations for m = 1, 2 and the row
  // and half exchanges for m = 4, 8, so that lanes with p a multiple of 2m
  // hold the pairwise sum of positions p .. p + 2m - 1 (the run's first
  // lanes, which store it, hold the run's).
  {
    const uint32_t rl = split / FK_ATTN_WAVES;  // a run's positions: 16 or 8
#pragma unroll
    for (uint32_t a = 0; a < HL; a++) {
      const uint32_t h = jq + 4 * a;
      if (a * 4 < group) {
        const float m = waves_max(sh.pm, min(h, group - 1));
        float w = 0.0f;
        if (h < group && r < n) w = exp_once(hs[a] - m);
        if (h < group && r < split) sh.wt[r * FK_ATTN_MAX_GROUP + h] = w;
        float t = w;
#pragma unroll
        for (uint32_t m2 = 1; m2 < FK_ATTN_MAX_SPLIT / FK_ATTN_WAVES; m2 <<= 1) {
          if (m2 >= rl) continue;
          if (m2 == 1) {
            t = t + dpp_f<0x12C>(t);  // row_ror:12: lane l + 4 of the row, position p + 1
          } else if (m2 == 2) {
            t = t + dpp_f<0x128>(t);  // row_ror:8: lane l + 8 of the row, position p + 2
          } else {
            const uint2 o = m2 == 4 ? rows_pair(__float_as_uint(t)) : halves_pair(__float_as_uint(t));
            t = __uint_as_float(o.x) + __uint_as_float(o.y);
          }
        }
        if (h < group && r < split && r % rl == 0) sh.pl[(r / rl) * FK_ATTN_MAX_GROUP + h] = t;
      }
    }
    // The values into LDS as the keys went (the new value row replacing row srow).
#pragma unroll
    for (int m = 0; m < 2; m++) {
      const uint32_t e = tid + m * T;
      const uint32_t rr = e / per_row;
      if (e < split * per_row && rr != srow) sh.vs[rr * per_row + e % per_row] = live2[m] ? vr[m] : u32x4{0u, 0u, 0u, 0u};
    }
    if (stores && tid < d) reinterpret_cast<uint16_t *>(sh.vs)[srow * d + tid] = vh;
  }
  __syncthreads();
  // Wavefront w's run of positions, lane i's dimension, every head at once.
  {
    constexpr uint32_t RUN_MAX = FK_ATTN_MAX_SPLIT / FK_ATTN_WAVES;
    const uint32_t run = split / FK_ATTN_WAVES;
    const uint32_t u0 = wave * run;
    float acc[FK_ATTN_MAX_GROUP];
#pragma unroll
    for (int h = 0; h < FK_ATTN_MAX_GROUP; h++) acc[h] = 0.0f;
    const uint32_t ic = min(lane, d - 1);
#pragma unroll
    for (uint32_t u = 0; u < RUN_MAX; u++) {
      if (u < run) {
        const float v = widen_cache(vsh[(u0 + u) * d + ic], bf16);
        const float4 w0 = *reinterpret_cast<const float4 *>(sh.wt + (u0 + u) * FK_ATTN_MAX_GROUP);
        const float4 w1 = group > 4 ? *reinterpret_cast<const float4 *>(sh.wt + (u0 + u) * FK_ATTN_MAX_GROUP + 4)
                                    : float4{0.0f, 0.0f, 0.0f, 0.0f};
        const float w[FK_ATTN_MAX_GROUP] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int h = 0; h < FK_ATTN_MAX_GROUP; h++)
          if ((uint32_t)h < group) acc[h] = __builtin_fmaf(w[h], v, acc[h]);
      }
    }
    // The keys were last read before the maxima's barrier: their LDS now holds
    // the runs' sums.
    float *pacc = reinterpret_cast<float *>(sh.ks);  // [wave][head][dim]
    if (lane < d) {
#pragma unroll
      for (int h = 0; h < FK_ATTN_MAX_GROUP; h++)
        if ((uint32_t)h < group) pacc[(wave * FK_ATTN_MAX_GROUP + h) * FK_ATTN_MAX_DIM + lane] = acc[h];
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
      const size_t ht = (size_t)(g * group + h) * p.splits + t;
      if (i == 0) {
        float *o = partials + (size_t)p.heads * p.splits * d + 2 * ht;
        o[0] = waves_max(sh.pm, h);
        o[1] = lt;
      }
      partials[ht * d + i] = at;
    }
  }
}

// The 1B decode's shape (groups of 4 query heads, heads of 64, splits of 128
// positions, f16 caches; a ring, or with PG paged pools): attend_split's
// arithmetic in the same order, with each wavefront's 16 positions (its run) in its registers
// from the keys' loads to the weighted values.  Thread (p, j) of wavefront w
// loads quarter j of position 16 w + p's key (32 bytes) and makes that
// position's scores; the values go into LDS as attend_split's do (while the
// scores are made), and lane i weighs dimension i of the run's rows by the
// run's weights, read from the lanes that made them.  Two barriers before the
// weighted values (the queries and the new rows; the heads' maxima and the
// values) and one before the runs' sums, where attend_split stages keys,
// weights and values in LDS between four.
template <bool PG>
__device__ __forceinline__ void attend_runs(AttendLds &sh, const float *__restrict__ q,
                                            const float *__restrict__ knew, const float *__restrict__ vnew,
                                            const CacheRows &cr, const uint32_t *__restrict__ position,
                                            const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                            float *__restrict__ partials, const uint32_t *__restrict__ reach,
                                            const fk_step_attend_params &p) {
  constexpr uint32_t G = 4, D = 64, S = 128, HALF = D / 2, RUN = S / FK_ATTN_WAVES;
  static_assert(RUN == 16 && FK_ATTN_WAVES * FK_WAVE == FK_ATTN_THREADS, "a wavefront's 16 positions are its run");
  uint16_t *__restrict__ kc = cr.kc;
  uint16_t *__restrict__ vc = cr.vc;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  const uint32_t g = blockIdx.x / p.splits;
  const uint32_t t = blockIdx.x % p.splits;
  const uint32_t pos = position[0];
  const uint32_t sraw = PG ? 0u : slot[0];
  const uint32_t s = sraw < p.slots ? sraw : 0;
  const uint32_t first = (p.window && pos + 1 > p.window) ? pos + 1 - p.window : 0;
  const uint32_t top = p.has_reach ? max(pos, reach[0]) : pos;
  const uint32_t lo = max(first, t * S);
  const uint32_t hi = min(top + 1, (t + 1) * S);
  const uint32_t n = hi > lo ? hi - lo : 0;
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  // A store needs its row's slot (a ring's) or block (a pool's) to exist.
  const bool held = PG ? (pos / cr.g.block_size < cr.g.table_len && slot[pos / cr.g.block_size] < cr.g.blocks)
                       : sraw < p.slots;
  const bool stores = p.store && held && lo <= pos && pos < hi;
  const uint32_t srow = stores ? pos - lo : 0xFFFFFFFFu;  // the split's row the new key and value replace
  const size_t base = ((size_t)s * p.kv_heads + g) * p.length;
  const uint32_t ring0 = PG ? 0u : lo % p.length;
  // Split row r's key and value rows (ring index (lo + r) mod length, or
  // position lo + r through the block table), a row past the split's
  // reading its last (or row lo) and replaced by zeros.
  auto row_of = [&](const uint16_t *c, const uint64_t *pool, uint32_t r) -> const uint16_t * {
    const uint32_t rr = min(r, n > 0 ? n - 1 : 0u);
    if constexpr (PG) {
      return paged_row(pool, slot, cr.g, lo + rr, g, D);
    } else {
      uint32_t ring = ring0 + rr;
      ring = ring >= p.length ? ring - p.length : ring;
      return c + (base + ring) * D;
    }
  };
  const uint32_t r = tid / 4;   // this thread's position of the split (its score's)
  const uint32_t jq = tid % 4;  // its quarter of the key, its head of the weights
  const uint32_t u0 = wave * RUN;

  // Loads, in the order their results are needed: the query rows with their
  // RoPE partners and cosines, the new rows, the key quarter, the values.
  float qx = 0.0f, qp = 0.0f, qc = 1.0f, qn = 0.0f;
  if (tid < G * D) {
    const float *head = q + (size_t)(g * G + tid / D) * D;
    const uint32_t j = tid % D;
    const uint32_t i = j < HALF ? j : j - HALF;
    qx = head[j];
    if (p.rope && i < p.rotated) {
      qp = head[j < HALF ? j + HALF : j - HALF];
      qc = cs[2 * i];
      qn = cs[2 * i + 1];
    }
  }
  float kx = 0.0f, kp = 0.0f, kcs = 1.0f, ksn = 0.0f, vx = 0.0f;
  if (stores && tid < D) {
    const float *head = knew + (size_t)g * D;
    const uint32_t j = tid;
    const uint32_t i = j < HALF ? j : j - HALF;
    kx = head[j];
    if (p.krope && i < p.rotated) {
      kp = head[j < HALF ? j + HALF : j - HALF];
      kcs = cs[2 * i];
      ksn = cs[2 * i + 1];
    }
    vx = vnew[(size_t)g * D + j];
  }
  const bool live = r < n;
  const u32x4 *krow = reinterpret_cast<const u32x4 *>(row_of(kc, cr.kpool, r) + 16 * jq);
  u32x4 kr[2];
  kr[0] = __builtin_nontemporal_load(krow);
  kr[1] = __builtin_nontemporal_load(krow + 1);
  // The values, 16 bytes a load: thread e's units e and e + 512 (row e / 8
  // and 64 rows on, unit e mod 8).
  u32x4 vr[2];
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint32_t e = tid + m * FK_ATTN_THREADS;
    vr[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(row_of(vc, cr.vpool, e / 8) + 8 * (e % 8)));
  }

  // The query rows RoPE'd into LDS; the new key row RoPE'd and the new value
  // row rounded into the cache, the key into LDS (the weights' LDS, unused
  // here) and the value into its row of the values' LDS.
  uint16_t *const knew_sh = reinterpret_cast<uint16_t *>(sh.wt);
  uint16_t *const vsh = reinterpret_cast<uint16_t *>(sh.vs);
  if (tid < G * D) {
    const uint32_t j = tid % D;
    const uint32_t i = j < HALF ? j : j - HALF;
    float v = qx;
    if (p.rope && i < p.rotated) v = j < HALF ? qx * qc - qp * qn : qx * qc + qp * qn;
    sh.qs[tid] = v;
  }
  if (stores && tid < D) {
    const uint32_t j = tid;
    const uint32_t i = j < HALF ? j : j - HALF;
    float k = kx;
    if (p.krope && i < p.rotated) k = j < HALF ? kx * kcs - kp * ksn : kx * kcs + kp * ksn;
    const uint16_t kh = narrow_cache(k, false);
    const uint16_t vh = narrow_cache(vx, false);
    if constexpr (PG) {
      paged_row(cr.kpool, slot, cr.g, pos, g, D)[j] = kh;
      paged_row(cr.vpool, slot, cr.g, pos, g, D)[j] = vh;
    } else {
      const size_t at = (base + pos % p.length) * D + j;
      kc[at] = kh;
      vc[at] = vh;
    }
    knew_sh[j] = kh;
    vsh[srow * D + j] = vh;
  }
  __syncthreads();

  // Scores: quarter jq of position r's key against every head's quarter,
  // the quad's chains added by DPP ((c0 + c1) + (c2 + c3)); lane 4 p + j
  // keeps head j's, and the wavefront's 16 positions give each head's
  // maximum into pm[head][wave].
  float hs;
  {
    uint32_t kw[8];
    if (r == srow) {
      const uint32_t *kn = reinterpret_cast<const uint32_t *>(knew_sh) + 8 * jq;
#pragma unroll
      for (int e = 0; e < 8; e++) kw[e] = kn[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        kw[e] = live ? kr[0][e] : 0u;
        kw[4 + e] = live ? kr[1][e] : 0u;
      }
    }
    float kf[16];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      kf[2 * e] = widen_cache((uint16_t)(kw[e] & 0xFFFFu), false);
      kf[2 * e + 1] = widen_cache((uint16_t)(kw[e] >> 16), false);
    }
    float sc[G];
#pragma unroll
    for (uint32_t h = 0; h < G; h++) {
      const float *qh = sh.qs + h * D + jq * 16;
      float c = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) c = __builtin_fmaf(qh[i], kf[i], c);
      c = c + dpp_f<0xB1>(c);  // quad_perm [1, 0, 3, 2]: c0 + c1, c2 + c3
      c = c + dpp_f<0x4E>(c);  // quad_perm [2, 3, 0, 1]: (c0 + c1) + (c2 + c3)
      sc[h] = live ? c * p.scale : -__builtin_inff();
    }
    hs = sc[0];
#pragma unroll
    for (uint32_t h = 1; h < G; h++) hs = jq == h ? sc[h] : hs;
    int k = max_key(hs);
    k = max(k, dpp_i<0x124>(k));  // row_ror:4
    k = max(k, dpp_i<0x128>(k));  // row_ror:8
    uint2 o = rows_pair((uint32_t)k);
    k = max((int)o.x, (int)o.y);
    o = halves_pair((uint32_t)k);
    k = max((int)o.x, (int)o.y);
    if (lane < G) sh.pm[lane * FK_ATTN_WAVES + wave] = from_max_key(k);
  }
  // The values into LDS (rows past the split's positions zero, the new row
  // already in its place).
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint32_t e = tid + m * FK_ATTN_THREADS;
    if (e / 8 != srow) sh.vs[e] = e / 8 < n ? vr[m] : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  // The weights exp(score - max) (zero past the split's positions) and the
  // run's pairwise sum of each head's (the tree of attend_split: lanes 0-3
  // hold the run's sums); then lane i's weighted values of the run, every
  // head at once, in order of position from +0, each weight read from the
  // lane that made it.
  const float w = live ? exp_once(hs - waves_max(sh.pm, jq)) : 0.0f;
  float tsum = w;
  tsum = tsum + dpp_f<0x12C>(tsum);  // row_ror:12: position p + 1
  tsum = tsum + dpp_f<0x128>(tsum);  // row_ror:8: position p + 2
  {
    uint2 o = rows_pair(__float_as_uint(tsum));
    tsum = __uint_as_float(o.x) + __uint_as_float(o.y);
    o = halves_pair(__float_as_uint(tsum));
    tsum = __uint_as_float(o.x) + __uint_as_float(o.y);
  }
  float acc[G];
#pragma unroll
  for (uint32_t h = 0; h < G; h++) acc[h] = 0.0f;
#pragma unroll
  for (uint32_t u = 0; u < RUN; u++) {
    const float v = widen_cache(vsh[(u0 + u) * D + lane], false);
#pragma unroll
    for (uint32_t h = 0; h < G; h++) {
      const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 4 * u + h));
      acc[h] = __builtin_fmaf(wu, v, acc[h]);
    }
  }
  float *pacc = reinterpret_cast<float *>(sh.ks);  // [wave][head][dim]
#pragma unroll
  for (uint32_t h = 0; h < G; h++) pacc[(wave * FK_ATTN_MAX_GROUP + h) * FK_ATTN_MAX_DIM + lane] = acc[h];
  if (lane < G) sh.pl[wave * FK_ATTN_MAX_GROUP + lane] = tsum;
  __syncthreads();
  if (tid < G * D) {
    const uint32_t h = tid / D;
    const uint32_t i = tid % D;
    float lt = 0.0f;
    float at = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < FK_ATTN_WAVES; w2++) {
      lt = lt + sh.pl[w2 * FK_ATTN_MAX_GROUP + h];
      at = at + pacc[(w2 * FK_ATTN_MAX_GROUP + h) * FK_ATTN_MAX_DIM + i];
    }
    const size_t ht = (size_t)(g * G + h) * p.splits + t;
    if (i == 0) {
      float *o = partials + (size_t)p.heads * p.splits * D + 2 * ht;
      o[0] = waves_max(sh.pm, h);
      o[1] = lt;
    }
    partials[ht * D + i] = at;
  }
}

}  // namespace fk

namespace fk {
// The attention launch's body (every kernel entry of it calls this): the
// shapes of the 1B decode specialised, every other shape general.
__device__ __forceinline__ void step_attend(const float *__restrict__ q, const float *__restrict__ knew,
                                            const float *__restrict__ vnew, uint16_t *__restrict__ kc,
                                            uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                                            const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                            float *__restrict__ partials, const uint32_t *__restrict__ reach,
                                            const fk_step_attend_params &p) {
  __shared__ AttendLds sh;
  const CacheRows cr{kc, vc, nullptr, nullptr, {1u, 1u, 1u}};
  const uint32_t group = p.heads / p.kv_heads;
  if (group == 4 && p.head_dim == 64 && p.split == 128 && !p.cache_bf16)
    attend_runs<false>(sh, q, knew, vnew, cr, position, slot, rope, partials, reach, p);
  else if (group == 4 && p.head_dim == 64 && p.split == 64 && !p.cache_bf16)
    attend_split<4, 64, 64, 0>(sh, q, knew, vnew, cr, position, slot, rope, partials, reach, p);
  else
    attend_split<0, 0, 0, -1>(sh, q, knew, vnew, cr, position, slot, rope, partials, reach, p);
}

// The attention over paged pools: kpool and vpool the blocks' addresses,
// `table` the row's block table.
__device__ __forceinline__ void step_attend_paged(const float *__restrict__ q, const float *__restrict__ knew,
                                                  const float *__restrict__ vnew, const uint64_t *__restrict__ kpool,
                                                  const uint64_t *__restrict__ vpool,
                                                  const uint32_t *__restrict__ position,
                                                  const uint32_t *__restrict__ table, const float *__restrict__ rope,
                                                  float *__restrict__ partials, const uint32_t *__restrict__ reach,
                                                  const fk_step_attend_paged_params &pp) {
  __shared__ AttendLds sh;
  const CacheRows cr{nullptr, nullptr, kpool, vpool, pp.g};
  const fk_step_attend_params &p = pp.a;
  const uint32_t group = p.heads / p.kv_heads;
  if (group == 4 && p.head_dim == 64 && p.split == 128 && !p.cache_bf16)
    attend_runs<true>(sh, q, knew, vnew, cr, position, table, rope, partials, reach, p);
  else
    attend_split<0, 0, 0, -1, true>(sh, q, knew, vnew, cr, position, table, rope, partials, reach, p);
}
}  // namespace fk


// Threadgroup (one wavefront) per head: M the largest of the splits' maxima
// (exact whatever the order), the splits' weights w_t = exp(max_t - M),
// binary64's rounded once, then lane i: out_i = (sum_t acc_t[i] w_t) /
// (sum_t l_t w_t), both sums in split order from +0.  Every load of a chunk of
// up to 64 splits is issued before any is used — the maxima and weight sums by
// lane t, the values acc_t[i] by lane i — so a chunk costs one round trip to
// memory; lane t makes split t's weight and l_t w_t and puts them in LDS,
// where the sums read them four at a time.
// The partials as the attention stores them: acc[heads][splits][head_dim],
// then [heads][splits][max, sum].
#define FK_COMBINE_CHUNK 64

namespace fk {

// One chunk of CH >= splits: every load first, each index clamped into the
// partials so that the compiler keeps them all in flight together.
template <int CH>
__device__ __forceinline__ void combine_chunk(const float *__restrict__ ph, const float *__restrict__ st,
                                              float *__restrict__ out, uint32_t head_dim, uint32_t splits,
                                              float *sw, float *slw) {
  const uint32_t lane = threadIdx.x;
  const uint32_t ic = min(lane, head_dim - 1);
  const uint32_t tc = min(lane, splits - 1);
  float mt = st[(size_t)tc * 2];
  const float lt = st[(size_t)tc * 2 + 1];
  float av[CH];
#pragma unroll
  for (int j = 0; j < CH; j++) av[j] = ph[(size_t)min((uint32_t)j, splits - 1) * head_dim + ic];
  if (lane >= splits) mt = -__builtin_inff();
  const float top = wave_max(mt);
  float wt = 0.0f, lw = 0.0f;
  if (lane < splits) {
    wt = exp_once(mt - top);
    lw = lt * wt;
  }
  sw[lane] = wt;
  slw[lane] = lw;
  __syncthreads();
  float l = 0.0f;
  float acc = 0.0f;
#pragma unroll
  for (int j4 = 0; j4 < CH / 4; j4++) {
    const float4 w4 = reinterpret_cast<const float4 *>(sw)[j4];
    const float4 l4 = reinterpret_cast<const float4 *>(slw)[j4];
    const float w[4] = {w4.x, w4.y, w4.z, w4.w};
    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
      if ((uint32_t)(4 * j4 + q) < splits) {
        l = l + lv[q];
        acc = acc + av[4 * j4 + q] * w[q];
      }
    }
  }
  if (lane < head_dim) out[lane] = acc / l;
}

}  // namespace fk

namespace fk {
// The combine launch's body (one wavefront a head).
__device__ __forceinline__ void step_combine(const float *__restrict__ partials, float *__restrict__ out,
                                             const fk_step_combine_params &p) {
  __shared__ float4 sw4[FK_COMBINE_CHUNK / 4], slw4[FK_COMBINE_CHUNK / 4];
  const uint32_t h = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  const uint32_t stride = p.head_dim;
  const float *ph = partials + (size_t)h * p.splits * stride;
  const float *st = partials + (size_t)p.heads * p.splits * stride + (size_t)h * p.splits * 2;
  if (p.splits <= FK_COMBINE_CHUNK && p.head_dim <= FK_WAVE) {
    float *o = out + (size_t)h * p.head_dim;
    if (p.splits <= 32)
      fk::combine_chunk<32>(ph, st, o, p.head_dim, p.splits, reinterpret_cast<float *>(sw4),
                            reinterpret_cast<float *>(slw4));
    else
      fk::combine_chunk<64>(ph, st, o, p.head_dim, p.splits, reinterpret_cast<float *>(sw4),
                            reinterpret_cast<float *>(slw4));
    return;
  }
  float m = -__builtin_inff();
  for (uint32_t t = lane; t < p.splits; t += FK_WAVE) m = fk::max_number(m, st[(size_t)t * 2]);
  const float top = fk::wave_max(m);
  for (uint32_t i0 = 0; i0 < p.head_dim; i0 += FK_WAVE) {
    const uint32_t i = i0 + lane;
    float l = 0.0f;
    float acc = 0.0f;
    for (uint32_t t0 = 0; t0 < p.splits; t0 += FK_COMBINE_CHUNK) {
      const uint32_t t = t0 + lane;
      float mt = 0.0f, lt = 0.0f;
      if (t < p.splits) {
        mt = st[(size_t)t * 2];
        lt = st[(size_t)t * 2 + 1];
      }
      float av[FK_COMBINE_CHUNK];
      const uint32_t ic = min(i, p.head_dim - 1);
#pragma unroll
      for (int j = 0; j < FK_COMBINE_CHUNK; j++) av[j] = ph[(size_t)min(t0 + j, p.splits - 1) * stride + ic];
      float wt = 0.0f, lw = 0.0f;
      if (t < p.splits) {
        wt = fk::exp_once(mt - top);
        lw = lt * wt;
      }
      float *sw = reinterpret_cast<float *>(sw4);
      float *slw = reinterpret_cast<float *>(slw4);
      __syncthreads();  // the last chunk's weights are read
      sw[lane] = wt;
      slw[lane] = lw;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < FK_COMBINE_CHUNK; j++) {
        if (t0 + j < p.splits) {
          l = l + slw[j];
          acc = acc + av[j] * sw[j];
        }
      }
    }
    if (i < p.head_dim) out[(size_t)h * p.head_dim + i] = acc / l;
  }
}
}  // namespace fk


// Wide splits ---------------------------------------------------------------
//
// The attention of one kv head's split of S = 64 W positions by W wavefronts
// of 64 positions each (W = blockDim / 64, up to 8), for splits few enough
// that the consumer of the partials (the combine, or the next GEMV step's
// prologue) reads them all cheaply.  Threadgroup (kv head g, split t); the
// partials' layout is the narrow kernel's.
//
// Lane l of wavefront w holds position r = t S + 64 w + l, its whole key and
// value rows in registers.  For query head h of the group:
//   score = (fma chain from +0 over the dimensions in order, q_i k_i) * scale
//           (-inf for a position off the split);
//   m_w   = the wave's maximumNumber of the scores (exact);
//   p     = exp(score - m_w) binary64's rounded once (0 if m_w is -inf);
//   l_w   = the pairwise sum of p over the 64 positions in order
//           ((p0 + p1) + (p2 + p3)) + ... (the wave_sum tree);
//   acc_w = for each dimension i, the fma chain from +0 of p_r v_r[i] over
//           the 64 positions in order.
// Then the threadgroup's: M the maximumNumber of the waves' m_w (exact);
// e_w = exp(m_w - M) binary64's rounded once (0 for a wave with no
// positions); L = sum over w in order from +0 of l_w e_w; A[i] = sum over w in
// order from +0 of acc_w[i] e_w (products rounded, then added).  A split
// with no positions stores M = -inf, L = 0, A = 0.
//
// The new key and value rows (if asked) are made by threads j < d, element j
// each, as the narrow kernel makes them, and the lane holding the position
// takes them from LDS.  Values of positions off the split are zeros in LDS
// (their weights are zero), so a cache's other contents never reach the sums.

#define FK_WIDE_MAX_WAVES 8
#define FK_WIDE_RUN 64
#define FK_WIDE_VT 68  // a transposed value row in LDS: 64 positions and 4 of padding

namespace fk {

// LDS of the wide attention, in floats: the queries [8][64], the new rows
// (64 halves each), the heads' maxima [8], then per wavefront the values
// transposed [32 pairs][68], the weights [8][64], the sums [8][64], the
// maxima and weight sums [8][2] and the waves' factors [8].
constexpr uint32_t WIDE_WAVE_FLOATS = 32 * FK_WIDE_VT + 8 * 64 + 8 * 64 + 16 + 8;
__host__ __device__ constexpr uint32_t wide_lds_floats(uint32_t waves) {
  return 512 + 64 + 8 + waves * WIDE_WAVE_FLOATS;
}

// R maxima at once, wave_max's steps interleaved.
template <int R>
__device__ __forceinline__ void wave_maxes(float (&x)[R]) {
  int v[R];
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = max_key(x[q]);
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = max(v[q], dpp_i<0xB1>(v[q]));
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = max(v[q], dpp_i<0x4E>(v[q]));
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = max(v[q], dpp_i<0x141>(v[q]));
#pragma unroll
  for (int q = 0; q < R; q++) v[q] = max(v[q], dpp_i<0x140>(v[q]));
#pragma unroll
  for (int q = 0; q < R; q++)
    x[q] = from_max_key(max(max(__builtin_amdgcn_readlane(v[q], 0), __builtin_amdgcn_readlane(v[q], 16)),
                            max(__builtin_amdgcn_readlane(v[q], 32), __builtin_amdgcn_readlane(v[q], 48))));
}

// One wavefront's 64 positions for the group's first R heads (R >= group):
// scores, maxima, weights and weight sums; the weights into et[h][lane].
template <int R>
__device__ __forceinline__ void wide_weights(const float *qs, const float (&kf)[64], uint32_t d, uint32_t group,
                                             bool live, float scale, float *et, float (&m)[R], float (&l)[R]) {
  const uint32_t lane = threadIdx.x & (FK_WAVE - 1);
#pragma unroll
  for (int h = 0; h < R; h++) {
    float c = 0.0f;
    if ((uint32_t)h < group) {
      const float4 *q4 = reinterpret_cast<const float4 *>(qs + h * d);
#pragma unroll
      for (int i4 = 0; i4 < 16; i4++) {
        if ((uint32_t)i4 < d / 4) {
          const float4 qv = q4[i4];
          c = __builtin_fmaf(qv.x, kf[4 * i4], c);
          c = __builtin_fmaf(qv.y, kf[4 * i4 + 1], c);
          c = __builtin_fmaf(qv.z, kf[4 * i4 + 2], c);
          c = __builtin_fmaf(qv.w, kf[4 * i4 + 3], c);
        }
      }
    }
    m[h] = live && (uint32_t)h < group ? c * scale : -__builtin_inff();
  }
  float sc[R];
#pragma unroll
  for (int h = 0; h < R; h++) sc[h] = m[h];
  wave_maxes<R>(m);
#pragma unroll
  for (int h = 0; h < R; h++) {
    l[h] = m[h] == -__builtin_inff() ? 0.0f : exp_once(sc[h] - m[h]);
    if ((uint32_t)h < group) et[h * 64 + lane] = l[h];
  }
  wave_sums<R>(l);
}

template <int CB>
__device__ __forceinline__ void attend_wide(const float *__restrict__ q, const float *__restrict__ knew,
                                            const float *__restrict__ vnew, uint16_t *__restrict__ kc,
                                            uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                                            const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                            float *__restrict__ partials, const uint32_t *__restrict__ reach,
                                            const fk_step_attend_params &p) {
  extern __shared__ float lds[];
  const uint32_t W = blockDim.x / FK_WAVE;
  float *qs = lds;                                                  // [group][d]
  uint16_t *kn = reinterpret_cast<uint16_t *>(lds + 512);          // [d]
  uint16_t *vn = kn + 64;                                           // [d]
  float *mm = lds + 512 + 64;                                       // [group]
  float *waves = lds + 512 + 64 + 8;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  float *wv = waves + (size_t)wave * WIDE_WAVE_FLOATS;
  uint32_t *vt = reinterpret_cast<uint32_t *>(wv);                  // [pair][FK_WIDE_VT]
  float *et = wv + 32 * FK_WIDE_VT;                                 // [h][64]

  const uint32_t g = blockIdx.x / p.splits;
  const uint32_t t = blockIdx.x % p.splits;
  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t d = p.head_dim;
  const uint32_t half = d / 2;
  const uint32_t S = p.split;
  const bool bf16 = CB >= 0 ? CB != 0 : p.cache_bf16 != 0;
  const uint32_t pos = position[0];
  const uint32_t sraw = slot[0];
  const uint32_t s = sraw < p.slots ? sraw : 0;
  const uint32_t first = (p.window && pos + 1 > p.window) ? pos + 1 - p.window : 0;
  const uint32_t lo = max(first, t * S);
  const uint32_t top = p.has_reach ? max(pos, reach[0]) : pos;
  const uint32_t hi = min(top + 1, (t + 1) * S);
  const bool stores = p.store && sraw < p.slots && lo <= pos && pos < hi;
  const float *cs = rope + (size_t)min(pos, p.rope_rows - 1) * 2 * p.rotated;
  const size_t base = ((size_t)s * p.kv_heads + g) * p.length;

  // This lane's position.
  const uint32_t at = t * S + FK_WIDE_RUN * wave + lane;
  const bool live = at >= lo && at < hi;
  const uint32_t ring = (live ? at : (hi > lo ? lo : 0)) % p.length;
  const uint16_t *krow = kc + (base + ring) * d;
  const uint16_t *vrow = vc + (base + ring) * d;

  // Loads first: the queries (and their RoPE partners and cosines), the new
  // rows' elements, then the lane's key and value rows, 16 bytes a load.
  float qx = 0.0f, qp = 0.0f, qc = 1.0f, qn = 0.0f;
  const uint32_t qj = tid % d;
  const uint32_t qi = qj < half ? qj : qj - half;
  if (tid < group * d) {
    const float *head = q + (size_t)(g * group + tid / d) * d;
    qx = head[qj];
    if (p.rope && qi < p.rotated) {
      qp = head[qj < half ? qj + half : qj - half];
      qc = cs[2 * qi];
      qn = cs[2 * qi + 1];
    }
  }
  float kx = 0.0f, kp = 0.0f, kcs = 1.0f, ksn = 0.0f, vx = 0.0f;
  if (stores && tid < d) {
    const float *head = knew + (size_t)g * d;
    kx = head[qj];
    if (p.krope && qi < p.rotated) {
      kp = head[qj < half ? qj + half : qj - half];
      kcs = cs[2 * qi];
      ksn = cs[2 * qi + 1];
    }
    vx = vnew[(size_t)g * d + qj];
  }
  u32x4 kr[8], vr[8];
#pragma unroll
  for (int c = 0; c < 8; c++) {
    if ((uint32_t)c < d / 8) {
      kr[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(krow) + c);
      vr[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vrow) + c);
    } else {
      kr[c] = vr[c] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  // The queries RoPE'd as rope_elem does, into LDS (a threadgroup of fewer
  // threads than the group's query elements takes the rest in more passes).
  if (tid < group * d) {
    float v = qx;
    if (p.rope && qi < p.rotated) v = qj < half ? qx * qc - qp * qn : qx * qc + qp * qn;
    qs[tid] = v;
  }
  for (uint32_t o = tid + blockDim.x; o < group * d; o += blockDim.x) {
    const float *head = q + (size_t)(g * group + o / d) * d;
    const uint32_t j = o % d;
    const uint32_t i = j < half ? j : j - half;
    float v = head[j];
    if (p.rope && i < p.rotated) {
      const float partner = head[j < half ? j + half : j - half];
      v = j < half ? v * cs[2 * i] - partner * cs[2 * i + 1] : v * cs[2 * i] + partner * cs[2 * i + 1];
    }
    qs[o] = v;
  }
  // The new rows, element tid: RoPE'd and rounded as the plan's store does,
  // into the caches and LDS.
  if (stores && tid < d) {
    float k = kx;
    if (p.krope && qi < p.rotated) k = qj < half ? kx * kcs - kp * ksn : kx * kcs + kp * ksn;
    const uint16_t kh = narrow_cache(k, bf16), vh = narrow_cache(vx, bf16);
    const size_t where = (base + pos % p.length) * d + qj;
    kc[where] = kh;
    vc[where] = vh;
    kn[qj] = kh;
    vn[qj] = vh;
  }
  __syncthreads();  // the queries and the new rows

  // The lane holding the position takes the new rows.
  if (stores && at == pos) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
      if ((uint32_t)c < d / 8) {
        kr[c] = reinterpret_cast<const u32x4 *>(kn)[c];
        vr[c] = reinterpret_cast<const u32x4 *>(vn)[c];
      }
    }
  }
  float kf[64];
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const uint32_t w4[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      kf[8 * c + 2 * e] = widen_cache((uint16_t)(w4[e] & 0xFFFFu), bf16);
      kf[8 * c + 2 * e + 1] = widen_cache((uint16_t)(w4[e] >> 16), bf16);
    }
  }
  // The values transposed into this wave's LDS, zeros off the split.
#pragma unroll
  for (int c = 0; c < 8; c++) {
    if ((uint32_t)c < d / 8) {
      vt[(4 * c) * FK_WIDE_VT + lane] = live ? vr[c].x : 0u;
      vt[(4 * c + 1) * FK_WIDE_VT + lane] = live ? vr[c].y : 0u;
      vt[(4 * c + 2) * FK_WIDE_VT + lane] = live ? vr[c].z : 0u;
      vt[(4 * c + 3) * FK_WIDE_VT + lane] = live ? vr[c].w : 0u;
    }
  }
  // Scores, maxima, weights (into et) and weight sums.
  float *aw = et + 8 * 64;  // [h][64]
  float *ml = aw + 8 * 64;  // [h][2]
  float *ew = ml + 16;      // [h]
  if (group <= 4) {
    float m[4], l[4];
    wide_weights<4>(qs, kf, d, group, live, p.scale, et, m, l);
    if (lane < 4) {
      ml[2 * lane] = lane == 0 ? m[0] : lane == 1 ? m[1] : lane == 2 ? m[2] : m[3];
      ml[2 * lane + 1] = lane == 0 ? l[0] : lane == 1 ? l[1] : lane == 2 ? l[2] : l[3];
    }
  } else {
    float m[8], l[8];
    wide_weights<8>(qs, kf, d, group, live, p.scale, et, m, l);
    if (lane < 8) {
      float mv = m[0], lv = l[0];
#pragma unroll
      for (int h = 1; h < 8; h++)
        if ((uint32_t)h == lane) mv = m[h], lv = l[h];
      ml[2 * lane] = mv;
      ml[2 * lane + 1] = lv;
    }
  }
  __syncthreads();  // the weights and values

  // The wave's weighted values: lane (a, j) = (lane / P, lane % P), P = d / 2
  // pairs, takes dimensions 2j and 2j + 1 of heads a, a + 64 / P, ...; four
  // positions a step, in order.
  {
    const uint32_t P = d / 2;
    const uint32_t jp = lane % P, a = lane / P, L = FK_WAVE / P;
    float acc[4][2];
#pragma unroll
    for (int k = 0; k < 4; k++) acc[k][0] = acc[k][1] = 0.0f;
    for (uint32_t p0 = 0; p0 < FK_WIDE_RUN; p0 += 4) {
      const u32x4 v4 = *reinterpret_cast<const u32x4 *>(vt + jp * FK_WIDE_VT + p0);
      const uint32_t vw[4] = {v4.x, v4.y, v4.z, v4.w};
      float vlo[4], vhi[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        vlo[e] = widen_cache((uint16_t)(vw[e] & 0xFFFFu), bf16);
        vhi[e] = widen_cache((uint16_t)(vw[e] >> 16), bf16);
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t h = a + k * L;
        if (h < group) {
          const float4 e4 = *reinterpret_cast<const float4 *>(et + h * 64 + p0);
          const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            acc[k][0] = __builtin_fmaf(ev[e], vlo[e], acc[k][0]);
            acc[k][1] = __builtin_fmaf(ev[e], vhi[e], acc[k][1]);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t h = a + k * L;
      if (h < group) *reinterpret_cast<float2 *>(aw + h * 64 + 2 * jp) = make_float2(acc[k][0], acc[k][1]);
    }
  }
  __syncthreads();  // every wave's sums, maxima and weight sums

  // The waves' factors: thread (w, h) takes e_w of head h, and wave 0's
  // threads the heads' maxima.
  if (tid < W * group) {
    const uint32_t w = tid / group, h = tid % group;
    int mk = max_key(-__builtin_inff());
    for (uint32_t u = 0; u < W; u++) mk = max(mk, max_key(waves[(size_t)u * WIDE_WAVE_FLOATS + 32 * FK_WIDE_VT +
                                                                 16 * 64 + 2 * h]));
    const float M = from_max_key(mk);
    float *mlw = waves + (size_t)w * WIDE_WAVE_FLOATS + 32 * FK_WIDE_VT + 16 * 64;
    const float mw = mlw[2 * h];
    mlw[16 + h] = mw == -__builtin_inff() ? 0.0f : exp_once(mw - M);
    if (w == 0) mm[h] = M;
  }
  __syncthreads();  // the factors

  // The threadgroup's partials.
  for (uint32_t o = tid; o < group * d; o += blockDim.x) {
    const uint32_t h = o / d, i = o % d;
    const float M = mm[h];
    float L = 0.0f, A = 0.0f;
    if (M != -__builtin_inff()) {
      for (uint32_t w = 0; w < W; w++) {
        const float *b = waves + (size_t)w * WIDE_WAVE_FLOATS + 32 * FK_WIDE_VT + 8 * 64;  // aw of wave w
        const float e = b[8 * 64 + 16 + h];
        L = L + b[8 * 64 + 2 * h + 1] * e;
        A = A + b[h * 64 + i] * e;
      }
    }
    const size_t ht = (size_t)(g * group + h) * p.splits + t;
    partials[ht * d + i] = A;
    if (i == 0) {
      float *st = partials + (size_t)p.heads * p.splits * d + 2 * ht;
      st[0] = M;
      st[1] = L;
    }
  }
}

__device__ __forceinline__ void step_attend_wide(const float *__restrict__ q, const float *__restrict__ knew,
                                                 const float *__restrict__ vnew, uint16_t *__restrict__ kc,
                                                 uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                                                 const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                                 float *__restrict__ partials, const uint32_t *__restrict__ reach,
                                                 const fk_step_attend_params &p) {
  if (p.cache_bf16)
    attend_wide<1>(q, knew, vnew, kc, vc, position, slot, rope, partials, reach, p);
  else
    attend_wide<0>(q, knew, vnew, kc, vc, position, slot, rope, partials, reach, p);
}

}  // namespace fk
