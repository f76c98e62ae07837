// fk_gemm.h — the prefill GEMM: C = A · Bᵀ on the matrix cores (gfx950 MFMA),
// the Linear anchors of a step of many rows (src/FuryKernel/Tile.hs:76-157:
// C = A·Bᵀ tiles staged in threadgroup memory; here f16 operands, binary32
// accumulation).
//
// Operands in HBM: A [M, K] (the step's input rows, rounded once to f16) and
// B [N, K] (the `out_in` weights, f16) both in the tile layout (fk_layout.h),
// so every load of a K step moves 1 KB of contiguous HBM straight into its
// place in LDS.  C is [M, ldc] f32 row-major, or for the SiLU·mul epilogue
// [M, N] f16 in the tile layout: the next GEMM's A.
//
// A threadgroup of 4 wavefronts (one a SIMD, each with the register file's
// whole share of 512) takes a 256 × 256 tile of C (for SiLU·mul, 256 rows ×
// 128 columns of gate and the same 128 of up, held together as one 256-row
// slab of the paired weights).  Wavefront (wm, wn) holds 128 × 128 of it as
// 8 × 8 blocks of 16 × 16 in AGPRs, accumulated by v_mfma_f32_16x16x32_f16:
// 64 matrix operations a wavefront each K step of 32, on 16 reads of 16
// bytes a lane from LDS.
//
// v_mfma_f32_16x16x32_f16 (D = A B + C, A 16 × 32, B 32 × 16): lane l holds
// A[l mod 16][8 (l div 16) .. + 7] and B[8 (l div 16) .. + 7][l mod 16] as 8
// halves each, and D[4 (l div 16) + r][l mod 16] as register r.  The
// weights are the first operand, so D's rows are C's columns and a lane
// holds four consecutive columns of one C row: 16-byte stores.  (The 16 × 16
// form rather than 32 × 32: a step's 64 operations have no dependence among
// them, and the shorter operations leave more places for the step's loads
// and reads between them; measured faster at every shape here.)
//
// The K loop is a ring of 4 LDS stages (4 × 32 KB), loaded by direct loads
// (buffer_load ... lds) 2 tiles ahead of the one being read; a step's loads,
// reads and matrix operations are interleaved, one barrier a step.
//
// The order of the sums over k is the matrix core's; results are held to the
// binary32 accumulation bound of the f16 products (the contract of Tile.hs's
// fragments), not to bits.
#pragma once

#include "fk_common.h"
#include "fk_layout.h"
#include "fk_mfma.h"

#define FK_GEMM_THREADS 256
#define FK_GEMM_BM 256
#define FK_GEMM_BN 256
#define FK_GEMM_BK 32
#ifndef FK_GEMM_STAGES
#define FK_GEMM_STAGES 4
#endif
#define FK_GEMM_LDS (FK_GEMM_STAGES * 2 * FK_GEMM_BM * FK_GEMM_BK * 2)
#define FK_LDS __attribute__((address_space(3)))

// The QKV epilogue's RoPE and caches (heads of 64, every pair turned).

// One threadgroup's tile.  MODE: the epilogue.
template <uint32_t MODE>
__device__ __forceinline__ void gemm_tile(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0,
                                          const _Float16 *__restrict__ b1, const _Float16 *__restrict__ b2,
                                          void *__restrict__ c0, void *__restrict__ c1, void *__restrict__ c2,
                                          const float *r0, const fk_gemm_params &p,
                                          const uint32_t *__restrict__ position = nullptr,
                                          const uint32_t *__restrict__ slot = nullptr,
                                          const float *__restrict__ rope = nullptr,
                                          const fk_gemm_rope_params &rp = fk_gemm_rope_params{},
                                          uint64_t *__restrict__ keys = nullptr,
                                          const fk_paging &pg = fk_paging{}) {
  extern __shared__ uint4 gemm_lds[];
  constexpr uint32_t ROW16 = FK_GEMM_BK * 2 / 16;           // 16-byte units a staged row takes
  constexpr uint32_t TILEB = FK_GEMM_BM * FK_GEMM_BK * 2;    // bytes of one operand's staged tile
  constexpr uint32_t STAGEB = 2 * TILEB;                     // a stage: A's tile, then B's
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (FK_WAVE - 1);
  const uint32_t wave = tid / FK_WAVE;
  const uint32_t wm = wave & 1;   // 128-row half of the tile
  const uint32_t wn = wave >> 1;  // 128-column half
  const uint32_t k = p.k;
  const uint32_t tiles_m = p.m / FK_GEMM_BM;
  const uint32_t tm = blockIdx.x % tiles_m;
  const uint32_t tn = blockIdx.x / tiles_m;
  const uint32_t m0 = tm * FK_GEMM_BM;

  // The weight slab of the tile: a plain tile's columns [n0, n0 + 256) of
  // one anchor; a SiLU·mul tile's slab tn of the pair, gate columns [n0, n0 +
  // 128) then the same up columns.
  uint32_t anchor = 0, n0;
  const _Float16 *bslab;
  if (MODE == FK_GEMM_SILU_MUL) {
    n0 = tn * (FK_GEMM_BN / 2);
    bslab = b0 + (size_t)tn * FK_GEMM_BN * k;
  } else {
    const uint32_t col = tn * FK_GEMM_BN;
    anchor = (p.n_anchors > 1 && col >= p.first_col[1] ? 1u : 0u) + (p.n_anchors > 2 && col >= p.first_col[2] ? 1u : 0u);
    n0 = col - (anchor == 0 ? p.first_col[0] : (anchor == 1 ? p.first_col[1] : p.first_col[2]));
    bslab = (anchor == 0 ? b0 : (anchor == 1 ? b1 : b2)) + (size_t)n0 * k;
  }

  // Tile loads.  A K step of an operand's slab is 16 KB of contiguous HBM in
  // its staged order; wave w loads chunks 4 w .. 4 w + 3 of each operand,
  // lane L's 16 bytes landing at unit L of the chunk.  One scalar descriptor
  // an operand slab, whose range ends the slab: no load reaches past it.
  const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t slab_bytes = FK_GEMM_BM * k * 2;
  const auto ra_src = fk::buffer(a + (size_t)m0 * k, slab_bytes);
  const auto rb_src = fk::buffer(bslab, slab_bytes);
  const uint32_t vl = wave_s * 4 * 1024 + lane * 16;
  FK_LDS char *const stage0 = (FK_LDS char *)gemm_lds + wave_s * 4 * 1024;

  // Fragment reads.  v_mfma_f32_16x16x32_f16 takes from lane l row l mod 16
  // of a 16-row block and k 8 (l div 16) .. + 7 of the step: a block is one
  // 1 KB chunk of the staged tile, lane l reading its row's logical unit
  // l div 16 at the swizzled place, and 16 lanes a cycle meet 16 different
  // bank groups.  A's blocks are rows wm 128 + 16 i of the tile; B's are
  // columns wn 128 + 16 j, or for SiLU·mul gate columns wn 64 + 16 j (blocks
  // 0-3) and the same up columns (blocks 4-7), so that a lane holds gate and
  // up of one element.
  const uint32_t lu = (lane % 16) * 4 + ((lane / 16) ^ fk::tile_swizzle(lane % 16));
  const uint32_t ra = wm * 8 * 64 + lu;
  const uint32_t rb = TILEB / 16 + (MODE == FK_GEMM_SILU_MUL ? wn * 4 : wn * 8) * 64 + lu;
#define FK_GEMM_BOFF(J) ((MODE == FK_GEMM_SILU_MUL && (J) >= 4 ? 4 + (J) : (J)) * 64)

  // 8 × 8 blocks of 16 × 16, 4 registers each: the 256 AGPRs.
  fk_float4v acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

  // Two sets of fragments (A's 8 blocks, B's 8).
  fk::Half8 fa0[8], fb0[8], fa1[8], fb1[8];
  // The fragments stay in VGPRs: the matrix operation would also take them
  // from AGPRs, and an allocation that puts them there moves accumulators
  // around the loop.  The constraint also completes their reads here.
#define FK_GEMM_PIN(X) asm volatile("" : "+v"((X).h))
  // The accumulators stay in AGPRs across steps: left free, the allocator
  // moves some of the 64 tuples through VGPRs every iteration.
#define FK_GEMM_PIN_ACC()                                                                                 \
  _Pragma("unroll") for (int i_ = 0; i_ < 8; i_++)                                                        \
  _Pragma("unroll") for (int j_ = 0; j_ < 8; j_++) asm volatile("" : "+a"(acc[i_][j_]))
#define FK_GEMM_MFMA_ROW(FA, FB, I)                                                                       \
  _Pragma("unroll") for (int j_ = 0; j_ < 8; j_++)                                                        \
    acc[I][j_] = __builtin_amdgcn_mfma_f32_16x16x32_f16(FB[j_].h, FA[I].h, acc[I][j_], 0, 0, 0)
  // s_waitcnt vmcnt(n), the other counters untouched (vmcnt's low four bits
  // at 3:0, its high two at 15:14).
#define FK_GEMM_VMCNT(N) __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (0x7 << 4) | (0xf << 8))
  // The workgroup barrier without the release fence of __syncthreads, which
  // would wait for every load in flight into LDS (vmcnt(0)); the loads this
  // barrier publishes are the ones the wait before it has seen land.  The
  // empty asm statements keep the compiler from moving LDS accesses across.
#define FK_GEMM_BARRIER()                 \
  do {                                    \
    asm volatile("" ::: "memory");        \
    __builtin_amdgcn_s_barrier();         \
    asm volatile("" ::: "memory");        \
  } while (0)
  // One K step of tile s (fragments FA, FB in registers; A's blocks 4-7
  // still on their way) in two halves of 32 matrix operations, A's blocks
  // 0-3 then 4-7 against all of B's.  The first half issues the loads of A's
  // part of tile s - 1 + S, and reads tile s + 1's B blocks and A blocks 0-3,
  // spread among its operations; the second completes the reads of FA's
  // blocks 4-7 (issued in the step before), issues B's loads and reads tile
  // s + 1's A blocks 4-7; the step ends completing the first half's reads.
  // So a read is waited for half a step after it goes out, the LDS sees the
  // step's reads spread over its matrix operations, and the address units
  // the loads the same way.
#define FK_GEMM_STEP(FA, FB, NA, NB, T_LOAD, ST_LOAD, ST_READ)                                           \
  do {                                                                                                    \
    FK_GEMM_VMCNT(8 * (FK_GEMM_STAGES - 3));                                                              \
    FK_GEMM_BARRIER();                                                                                    \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    const uint32_t so_ = (T_LOAD) * TILEB;                                                                \
    FK_LDS char *d_ = stage0 + (ST_LOAD) * STAGEB;                                                        \
    const uint4 *s_ = gemm_lds + (ST_READ) * (STAGEB / 16);                                               \
    _Pragma("unroll") for (int q = 0; q < 4; q++) {                                                       \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_src, d_ + q * 1024, 16, vl + q * 1024, so_, 0, 0);      \
      NB[2 * q].u = s_[rb + FK_GEMM_BOFF(2 * q)];                                                         \
      NB[2 * q + 1].u = s_[rb + FK_GEMM_BOFF(2 * q + 1)];                                                 \
      NA[q].u = s_[ra + 64 * q];                                                                          \
    }                                                                                                     \
    _Pragma("unroll") for (int i_ = 0; i_ < 4; i_++) { FK_GEMM_MFMA_ROW(FA, FB, i_); }                    \
    _Pragma("unroll") for (int g_ = 0; g_ < 4; g_++) {                                                    \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                  \
    }                                                                                                     \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    _Pragma("unroll") for (int i_ = 4; i_ < 8; i_++) FK_GEMM_PIN(FA[i_]);                                 \
    _Pragma("unroll") for (int q = 0; q < 4; q++) {                                                       \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_src, d_ + TILEB + q * 1024, 16, vl + q * 1024, so_, 0, 0); \
      NA[4 + q].u = s_[ra + 64 * (4 + q)];                                                                \
    }                                                                                                     \
    _Pragma("unroll") for (int i_ = 4; i_ < 8; i_++) { FK_GEMM_MFMA_ROW(FA, FB, i_); }                    \
    _Pragma("unroll") for (int g_ = 0; g_ < 4; g_++) {                                                    \
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                  \
    }                                                                                                     \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    _Pragma("unroll") for (int j_ = 0; j_ < 8; j_++) FK_GEMM_PIN(NB[j_]);                                 \
    _Pragma("unroll") for (int i_ = 0; i_ < 4; i_++) FK_GEMM_PIN(NA[i_]);                                 \
    FK_GEMM_PIN_ACC();                                                                                    \
  } while (0)

  // The pipeline, S = STAGES deep.  At step s (after its barrier) tile s's
  // fragments are in registers but for A's blocks 4-7, on the way from LDS
  // stage s mod S, and tiles s + 1 .. s + S - 2 are in their stages (numbers
  // mod S) or on their way there.  Step s waits for its own loads of tile s
  // + 1, meets the others at the barrier (after which all of tile s + 1 is in
  // LDS and every wave has completed its reads of tile s - 1), loads tile s -
  // 1 + S into tile s - 1's stage, reads tile s + 1's fragments and
  // multiplies tile s's.  Loads past the last tile repeat it into stages no
  // step reads, so every step's wait counts the same loads.
  const uint32_t steps = k / FK_GEMM_BK;  // even
  const uint32_t last = steps - 1;
#define FK_GEMM_T(X) ((X) < last ? (X) : last)
#pragma unroll
  for (uint32_t t = 0; t + 1 < FK_GEMM_STAGES; t++) {
    const uint32_t so_ = FK_GEMM_T(t) * TILEB;
    FK_LDS char *d_ = stage0 + t * STAGEB;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_src, d_ + q * 1024, 16, vl + q * 1024, so_, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_src, d_ + TILEB + q * 1024, 16, vl + q * 1024, so_, 0, 0);
    }
  }
  FK_GEMM_VMCNT(8 * (FK_GEMM_STAGES - 2));  // tile 0 landed
  FK_GEMM_BARRIER();
#pragma unroll
  for (int q = 0; q < 8; q++) {
    fb0[q].u = gemm_lds[rb + FK_GEMM_BOFF(q)];
    fa0[q].u = gemm_lds[ra + 64 * q];
  }
#pragma unroll
  for (int q = 0; q < 8; q++) FK_GEMM_PIN(fb0[q]);
#pragma unroll
  for (int q = 0; q < 4; q++) FK_GEMM_PIN(fa0[q]);
  for (uint32_t s = 0; s < steps; s += 2) {
    FK_GEMM_STEP(fa0, fb0, fa1, fb1, FK_GEMM_T(s - 1 + FK_GEMM_STAGES), (s + FK_GEMM_STAGES - 1) % FK_GEMM_STAGES,
                 (s + 1) % FK_GEMM_STAGES);
    FK_GEMM_STEP(fa1, fb1, fa0, fb0, FK_GEMM_T(s + FK_GEMM_STAGES), s % FK_GEMM_STAGES, (s + 2) % FK_GEMM_STAGES);
  }
  // Nothing may still be landing in LDS when the threadgroup ends.
  __builtin_amdgcn_s_waitcnt(0);
#undef FK_GEMM_PIN
#undef FK_GEMM_PIN_ACC
#undef FK_GEMM_MFMA_ROW
#undef FK_GEMM_VMCNT
#undef FK_GEMM_BARRIER
#undef FK_GEMM_STEP
#undef FK_GEMM_T
#undef FK_GEMM_BOFF

  // Epilogue.  Block (i, j)'s lane l holds C row m = wm 128 + 16 i + l mod 16
  // and columns 16 j + 4 (l div 16) .. + 3 (of the wavefront's).  (The lane
  // index is taken anew through an asm statement, so that nothing of the
  // epilogue is computed before the loop and held in registers across it.)
  uint32_t lane_e;
  asm volatile("v_mov_b32 %0, %1" : "=v"(lane_e) : "v"(lane));
  const uint32_t m = m0 + wm * 128 + lane_e % 16;
  const uint32_t nq = 4 * (lane_e / 16);
  if (MODE == FK_GEMM_SILU_MUL) {
    uint16_t *out = reinterpret_cast<uint16_t *>(c0);
    const uint32_t ncols = p.ldc[0];
    // silu(g) u = g / (1 + e^-g) · u, or gelu(g) u = 0.5 g (1 + tanh(y)) u
    // with tanh(y) = 1 - 2 / (1 + e^2y), with the hardware's exp and
    // reciprocal (a few ulp of binary32), then rounded once to f16 (2^-11):
    // the f16 rounding bounds the error.  An exponential overflowing gives
    // the limits (silu 0, tanh 1).  The activation is a branch on the
    // launch's uniform parameter around the whole epilogue, each side
    // unrolled, so a tile pays for its own activation's exponentials only.
    auto act_mul_tiles = [&](auto gelu_tag) {
      constexpr bool GELU = decltype(gelu_tag)::value;
#pragma unroll
      for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          // Blocks 0-3: gate columns wn 64 + 16 j; blocks 4-7 the same up columns.
          const uint32_t n = n0 + wn * 64 + 16 * j + nq;
          uint16_t h[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float gt = acc[i][j][r];
            const float u = acc[i][j + 4][r];
            float a;
            if constexpr (GELU) {
              const float y = 0.7978845608028654f * (gt + ((0.044715f * gt) * gt) * gt);
              const float th = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(2.0f * y));
              a = (0.5f * gt) * (1.0f + th);
            } else {
              a = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt));
            }
            h[r] = fk::to_f16(a * u);
          }
          uint2 w;
          w.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
          w.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
          // Four consecutive columns of one row: half of one 16-byte unit.
          *reinterpret_cast<uint2 *>(out + fk::tile_offset(m + 16 * i, n, ncols)) = w;
          if (j == 3) asm volatile("" ::: "memory");  // one row block at a time
        }
    };
    if (p.act == FK_ACT_GELU_TANH) act_mul_tiles(fk_bool_tag<true>{});
    else act_mul_tiles(fk_bool_tag<false>{});
  } else if (MODE == FK_GEMM_QKV_ROPE || MODE == FK_GEMM_QKV_ROPE_PAGED) {
    // A 256-column tile is 4 whole heads, a wavefront's 128 columns 2; a
    // lane's blocks 4 jp + jj and 4 jp + jj + 2 hold columns d and d + 32 of
    // head jp, both elements of each pair RoPE turns (NeoX halves, as
    // rope_elem: x_j c - x_{j+32} s below the half, x_j c + x_{j-32} s above,
    // the table's cos and sin of the row's position).  q goes to f16 rows
    // (the attention's), k and v to the caches.  Every choice is uniform and
    // made by selects, with the hardware's f16 conversion (to nearest even,
    // gradual underflow: narrow_f16's rounding), so the row-block loop
    // unrolls and the accumulators stay in registers.
    const bool bf16 = rp.cache_bf16 != 0;
    const bool turn = anchor != 2;
    const uint32_t head0 = (n0 + wn * 128) / 64;
    uint16_t *const dst = reinterpret_cast<uint16_t *>(anchor == 0 ? c0 : (anchor == 1 ? c1 : c2));
    // halves from head to head: q's rows and staged k, v rows hold a row's
    // heads side by side, a ring a head's length positions apart, a paged
    // pool's block a block's positions apart
    constexpr bool PAGED = MODE == FK_GEMM_QKV_ROPE_PAGED;
    const size_t hstride = anchor == 0 || rp.staged ? 64 : (PAGED ? (size_t)pg.block_size : (size_t)rp.length) * 64;
    // Row block i's RoPE and stores: `base` its row's first head, `unit(u)`
    // the u-th 16 bytes (pairs 2 u, 2 u + 1) of its position's table row.
    auto emit = [&](int i, uint16_t *const base, bool keep, auto unit) {
#pragma unroll
      for (int jp = 0; jp < 2; jp++)
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
          const uint32_t d = 16 * jj + nq;  // the low half's first of four columns; their partners d + 32 ..
          const float4 t01 = unit(d / 2);      // (cos, sin) of pairs d, d + 1
          const float4 t23 = unit(d / 2 + 1);  // pairs d + 2, d + 3
          const float cc[4] = {t01.x, t01.z, t23.x, t23.z};
          const float sn[4] = {t01.y, t01.w, t23.y, t23.w};
          uint16_t lo[4], hi[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float x = acc[i][4 * jp + jj][r], y = acc[i][4 * jp + jj + 2][r];
            const float xr = turn ? x * cc[r] - y * sn[r] : x;
            const float yr = turn ? y * cc[r] + x * sn[r] : y;
            lo[r] = bf16 && anchor != 0 ? fk::narrow_bf16(xr) : fk::to_f16(xr);
            hi[r] = bf16 && anchor != 0 ? fk::narrow_bf16(yr) : fk::to_f16(yr);
          }
          uint16_t *const at = base + jp * hstride + d;
          if (keep) {
            *reinterpret_cast<uint2 *>(at) =
                make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
            *reinterpret_cast<uint2 *>(at + 32) =
                make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
          }
        }
      asm volatile("" ::: "memory");  // one row block at a time
    };
    if constexpr (PAGED) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t row = m + 16 * i;
        const uint32_t pos = position[row];
        // `slot` holds the rows' block tables; position pos's block, the
        // table index and the block clamped into place.  A position past its
        // table stores no k or v (as the decode step's paged store skips
        // it); its q row is still written.
        const uint32_t sl =
            min(slot[(size_t)row * pg.table_len + min(pos / pg.block_size, pg.table_len - 1)], pg.blocks - 1);
        const bool keep = anchor == 0 || pos / pg.block_size < pg.table_len;
        const float *cs = rope + (size_t)min(pos, rp.rope_rows - 1) * 64;
        uint16_t *const base =
            anchor == 0 ? dst + (size_t)row * p.ldc[0] + head0 * 64
                        : dst + (((size_t)sl * rp.kv_heads + head0) * pg.block_size + pos % pg.block_size) * 64;
        emit(i, base, keep, [&](uint32_t u) { return *reinterpret_cast<const float4 *>(cs + 4 * u); });
      }
    } else {
      // A ring's tile: its 256 rows' RoPE table entries and ring places go
      // into LDS first (the K loop's ring is free once every wavefront is
      // past its last step), and the row blocks read them there: read from
      // HBM at each row block's turn, every row block would wait for its
      // loads behind the stores of the row block before it (the vector
      // memory counter counts loads and stores together).  Thread t takes row
      // t's position and place (the offset of its first head's row in the
      // ring); then each wavefront loads 64 rows' entries straight into LDS,
      // 4 rows (1 KB) a load, lane L taking 16-byte unit (L mod 16) ^ (r mod
      // 16) of row r = 4 q + L div 16 into place L mod 16 of the row, so that
      // the 16 rows of a row block's reads meet 16 different places.
      float *const lrope = reinterpret_cast<float *>(gemm_lds);  // [256 rows][64]
      uint32_t *const lpos = reinterpret_cast<uint32_t *>(lrope + 256 * 64);
      uint64_t *const lrow = reinterpret_cast<uint64_t *>(lpos + 256);
      __syncthreads();
      {
        const uint32_t row = m0 + tid;
        const uint32_t pos = position[row];
        lpos[tid] = min(pos, rp.rope_rows - 1);
        // (The ring length is taken anew through an asm statement, so that
        // its reciprocal is not computed before the K loop and held across
        // it.)
        uint32_t length = rp.length;
        asm volatile("" : "+s"(length));
        lrow[tid] = ((uint64_t)min(slot[row], rp.slots - 1) * rp.kv_heads * length + pos % length) * 64;
      }
      __syncthreads();
      {
        const auto rsrc = fk::buffer(rope, (size_t)rp.rope_rows * 64 * 4);
        FK_LDS char *const lbase = (FK_LDS char *)gemm_lds + wave_s * 64 * 256;
#pragma unroll
        for (int q = 0; q < 16; q++) {
          const uint32_t r = wave * 64 + 4 * q + lane / 16;
          const uint32_t unit = (lane % 16) ^ (r % 16);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lbase + q * 1024, 16, (lpos[r] * 64 + unit * 4) * 4, 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t rt = wm * 128 + lane_e % 16 + 16 * i;  // the row in the tile
        const uint32_t row = m0 + rt;
        const float *cs = lrope + rt * 64;
        uint16_t *const base = anchor == 0 ? dst + (size_t)row * p.ldc[0] + head0 * 64
                               : rp.staged ? dst + ((size_t)row * rp.kv_heads + head0) * 64
                                           : dst + lrow[rt] + head0 * hstride;
        emit(i, base, true,
             [&](uint32_t u) { return *reinterpret_cast<const float4 *>(cs + 4 * (u ^ (rt % 16))); });
      }
    }
  } else {
    float *out = reinterpret_cast<float *>(anchor == 0 ? c0 : (anchor == 1 ? c1 : c2));
    const uint32_t ld = anchor == 0 ? p.ldc[0] : (anchor == 1 ? p.ldc[1] : p.ldc[2]);
    // The greedy token's keys (one anchor, its columns from 0): the key of
    // the largest element of each row's 128 columns of the wavefront, the
    // row's key part (n0 + wn 128) / 128 of ld / 128.  A lane meets its
    // columns in increasing order and keeps the first of its largest by the
    // high word of fk::argmax_key alone (the value's order: NaN 0 but at
    // column 0, where it is above everything), so the 64-bit key is made
    // once a row block, from the kept value and column.
    const uint32_t col0 = n0 + wn * 128 + nq;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const size_t row = (size_t)(m + 16 * i) * ld + n0 + wn * 128 + nq;
      uint32_t bk = 0, bi = col0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        fk_float4v v = acc[i][j];
        if (MODE == FK_GEMM_ADD) v = *reinterpret_cast<const fk_float4v *>(r0 + row + 16 * j) + v;
        else {
          // Through an arithmetic copy (the canonical value: the same number):
          // a store straight from the accumulator leaves the allocator free
          // to hold accumulators in VGPRs through the loop, copying them at
          // every step.
#pragma unroll
          for (int r = 0; r < 4; r++) v[r] = __builtin_canonicalizef(v[r]);
        }
        if (MODE == FK_GEMM_STORE_KEYS) {
          // The logits: a gigabyte no later launch of the step reads (the
          // keys carry the token), streamed past the caches.
          __builtin_nontemporal_store(v, reinterpret_cast<fk_float4v *>(out + row + 16 * j));
        } else {
          *reinterpret_cast<fk_float4v *>(out + row + 16 * j) = v;
        }
        if (MODE == FK_GEMM_STORE_KEYS) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float z = v[r] + 0.0f;  // -0 to +0: the two zeros are one value
            const uint32_t u = __float_as_uint(z);
            const uint32_t nan_key = j == 0 && r == 0 && col0 == 0 ? 0xFFFFFFFFu : 0u;
            const uint32_t key = z != z ? nan_key : u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
            bi = key > bk ? col0 + 16 * j + r : bi;
            bk = key > bk ? key : bk;
          }
        }
      }
      if (MODE == FK_GEMM_STORE_KEYS) {
        uint64_t best = ((uint64_t)bk << 32) | (uint64_t)(0xFFFFFFFFu - bi);
        // Lanes l, l ^ 16, l ^ 32 and l ^ 48 hold the same row's other
        // columns of the wavefront's 128.
#pragma unroll
        for (int s = 16; s <= 32; s <<= 1) {
          const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(best >> 32), s) << 32) |
                                 (uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)best, s);
          best = other > best ? other : best;
        }
        if (lane_e < 16) keys[(size_t)(m + 16 * i) * (ld / 128) + (n0 + wn * 128) / 128] = best;
      }
      // One row block at a time: the compiler may not gather every block's
      // addresses (and loads) ahead, which would crowd the registers the
      // accumulators hold.
      asm volatile("" ::: "memory");
    }
  }
}

// Buffers in binding order, then the parameter struct.  The grid: one
// threadgroup a tile, tiles of 256 rows down M first.
#define FK_GEMM_ENTRY(NAME, MODE)                                                                                   \
  extern "C" __global__ void __launch_bounds__(FK_GEMM_THREADS)                                                     \
      NAME(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0, const _Float16 *__restrict__ b1,      \
           const _Float16 *__restrict__ b2, void *__restrict__ c0, void *__restrict__ c1, void *__restrict__ c2,   \
           const float *r0, fk_gemm_params p) {                                                                    \
    gemm_tile<MODE>(a, b0, b1, b2, c0, c1, c2, r0, p);                                                            \
  }

FK_GEMM_ENTRY(fk_gemm_f16_store, FK_GEMM_STORE)
FK_GEMM_ENTRY(fk_gemm_f16_add, FK_GEMM_ADD)
FK_GEMM_ENTRY(fk_gemm_f16_silu_mul, FK_GEMM_SILU_MUL)

// The plain store with the greedy token folded in: one anchor, its C rows
// and each row's keys [M][N / 128], which fk_prefill_argmax_keys reduces.
extern "C" __global__ void __launch_bounds__(FK_GEMM_THREADS)
    fk_gemm_f16_store_keys(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0,
                           const _Float16 *__restrict__ b1, const _Float16 *__restrict__ b2, void *__restrict__ c0,
                           void *__restrict__ c1, void *__restrict__ c2, const float *r0, uint64_t *__restrict__ keys,
                           fk_gemm_params p) {
  gemm_tile<FK_GEMM_STORE_KEYS>(a, b0, b1, b2, c0, c1, c2, r0, p, nullptr, nullptr, nullptr, fk_gemm_rope_params{},
                                keys);
}

// The QKV projection with RoPE and the KV store in its epilogue: anchors q,
// k, v (in that order), C0 the f16 q rows, C1 and C2 the K and V caches
// ([slots][kv_heads][length][64]), then each row's position and slot and the
// RoPE table ([position][32 pairs][cos, sin]).
extern "C" __global__ void __launch_bounds__(FK_GEMM_THREADS)
    fk_gemm_f16_qkv_rope(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0,
                         const _Float16 *__restrict__ b1, const _Float16 *__restrict__ b2, void *__restrict__ c0,
                         void *__restrict__ c1, void *__restrict__ c2, const float *r0,
                         const uint32_t *__restrict__ position, const uint32_t *__restrict__ slot,
                         const float *__restrict__ rope, fk_gemm_qkv_params p) {
  gemm_tile<FK_GEMM_QKV_ROPE>(a, b0, b1, b2, c0, c1, c2, r0, p.g, position, slot, rope, p.r);
}

// The same with the K and V caches paged pools ([blocks][kv_heads][block
// size][64]) and `table` the rows' block tables ([rows][table_len]).
extern "C" __global__ void __launch_bounds__(FK_GEMM_THREADS)
    fk_gemm_f16_qkv_rope_paged(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0,
                               const _Float16 *__restrict__ b1, const _Float16 *__restrict__ b2, void *__restrict__ c0,
                               void *__restrict__ c1, void *__restrict__ c2, const float *r0,
                               const uint32_t *__restrict__ position, const uint32_t *__restrict__ table,
                               const float *__restrict__ rope, fk_gemm_qkv_paged_params p) {
  gemm_tile<FK_GEMM_QKV_ROPE_PAGED>(a, b0, b1, b2, c0, c1, c2, r0, p.g, position, table, rope, p.r, nullptr, p.pg);
}
