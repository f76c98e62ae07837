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
template <uint32_t G, uint32_t D, uint32_t S, int CB>
__device__ __forceinline__ void attend_split(AttendLds &sh, const float *__restrict__ q,
                                             const float *__restrict__ knew, const float *__restrict__ vnew,
                                             uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                             const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot,
                                             const float *__restrict__ rope, float *__restrict__ partials,
                                             const fk_step_attend_params &p) {
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
  // The row the new key and value replace (none unless this split stores).
  const uint32_t srow = stores ? pos - lo : 0xFFFFFFFFu;
  // The split's keys, then its values, 16 bytes a load, non-temporal (a step
  // reads each cached row once): K is staged before the scores, V while they
  // are made.  Every load unconditional, a chunk past the split's rows
  // reading its last chunk (or the ring's row lo) and replaced by zeros.
  size_t at2[2];
  bool live2[2];
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint32_t e = tid + m * T;
    live2[m] = e < chunks;
    const uint32_t ec = min(e, chunks > 0 ? chunks - 1 : 0u);
    uint32_t ring = ring0 + ec / per_row;
    ring = ring >= p.length ? ring - p.length : ring;
    at2[m] = (base + ring) * d + 8 * (ec % per_row);
  }
  u32x4 kr[2], vr[2];
#pragma unroll
  for (int m = 0; m < 2; m++) kr[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kc + at2[m]));
#pragma unroll
  for (int m = 0; m < 2; m++) vr[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vc + at2[m]));

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
    const size_t at = (base + pos % p.length) * d + j;
    kc[at] = kh;
    vc[at] = vh;
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
        k = max(k, __shfl_xor(k, 16));
        k = max(k, __shfl_xor(k, 32));
        if (lane < 4 && a * 4 + lane < group) sh.pm[(a * 4 + lane) * FK_ATTN_WAVES + wave] = from_max_key(k);
      }
    }
  }
  __syncthreads();
  // The weights exp(score - max), the head's maximum the largest of the
  // wavefronts': thread (r, j) makes heads j and j + 4 (zero past the
  // positions the split holds), then each run's pairwise sum over its
  // positions by shuffles (lane 4p + j's partner at level m holds position
  // p ^ m, same head).
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
        for (uint32_t m2 = 1; m2 < FK_ATTN_MAX_SPLIT / FK_ATTN_WAVES; m2 <<= 1)
          if (m2 < rl) t = t + __shfl_xor(t, 4 * m2);
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

}  // namespace fk

namespace fk {
// The attention launch's body (every kernel entry of it calls this): the
// shapes of the 1B decode specialised, every other shape general.
__device__ __forceinline__ void step_attend(const float *__restrict__ q, const float *__restrict__ knew,
                                            const float *__restrict__ vnew, uint16_t *__restrict__ kc,
                                            uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
                                            const uint32_t *__restrict__ slot, const float *__restrict__ rope,
                                            float *__restrict__ partials, const fk_step_attend_params &p) {
  __shared__ AttendLds sh;
  const uint32_t group = p.heads / p.kv_heads;
  if (group == 4 && p.head_dim == 64 && p.split == 128 && !p.cache_bf16)
    attend_split<4, 64, 128, 0>(sh, q, knew, vnew, kc, vc, position, slot, rope, partials, p);
  else if (group == 4 && p.head_dim == 64 && p.split == 64 && !p.cache_bf16)
    attend_split<4, 64, 64, 0>(sh, q, knew, vnew, kc, vc, position, slot, rope, partials, p);
  else
    attend_split<0, 0, 0, -1>(sh, q, knew, vnew, kc, vc, position, slot, rope, partials, p);
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

