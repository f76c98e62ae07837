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
// 4 × 4 blocks of 32 × 32 in AGPRs, accumulated by v_mfma_f32_32x32x16_f16:
// 32 matrix operations a wavefront each K step of 32, on 16 reads of 16
// bytes a lane from LDS.
//
// v_mfma_f32_32x32x16_f16 (D = A B + C, A 32 × 16, B 16 × 32): lane l holds
// A[l mod 32][8 (l div 32) .. + 7] and B[8 (l div 32) .. + 7][l mod 32] as 8
// halves each, and D[8 g + 4 (l div 32) + r][l mod 32] as register 4 g + r.
// The weights are the first operand, so D's rows are C's columns and a lane
// holds four consecutive columns of one C row: 16-byte stores.
//
// The K loop is a ring of 4 LDS stages (4 × 32 KB): tiles go in 3 steps
// ahead by direct loads (buffer_load ... lds), the fragments of the next
// step are read while this step's are multiplied, one barrier a step.
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
#define FK_GEMM_STAGES 4
#define FK_GEMM_LDS (FK_GEMM_STAGES * 2 * FK_GEMM_BM * FK_GEMM_BK * 2)
#define FK_LDS __attribute__((address_space(3)))


enum : uint32_t {
  FK_GEMM_STORE = 0,     // C = A Bᵀ (f32 rows)
  FK_GEMM_ADD = 1,       // C = R + A Bᵀ (f32 rows), R [M, ldc]; R may be C
  FK_GEMM_SILU_MUL = 2,  // C = f16(silu(A Gᵀ) · (A Uᵀ)) in the tile layout; B0 the paired gate/up weights
  FK_GEMM_QKV_ROPE = 3,  // anchors q, k, v: q RoPE'd into f16 rows (C0), k RoPE'd into the K cache (C1), v
                         // into the V cache (C2), at each row's slot and position
};

struct fk_gemm_params {
  uint32_t m;            // rows of A and C, a multiple of 256
  uint32_t k;            // a multiple of 64
  uint32_t n_anchors;    // 1 to 3 weights (SiLU·mul: 1, the pair)
  uint32_t first_col[4]; // anchor j's columns of C are [first_col[j], first_col[j + 1]), each a multiple of 256
  uint32_t ldc[3];       // row stride of anchor j's output (its columns; SiLU·mul: N, gate's rows)
};

// The QKV epilogue's RoPE and caches (heads of 64, every pair turned).
struct fk_gemm_rope_params {
  uint32_t kv_heads;
  uint32_t rope_rows;    // positions the RoPE table holds
  uint32_t length;       // ring length
  uint32_t slots;
  uint32_t cache_bf16;
};

struct fk_gemm_qkv_params {
  fk_gemm_params g;
  fk_gemm_rope_params r;
};

// One threadgroup's tile.  MODE: the epilogue.
template <uint32_t MODE>
__device__ __forceinline__ void gemm_tile(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0,
                                          const _Float16 *__restrict__ b1, const _Float16 *__restrict__ b2,
                                          void *__restrict__ c0, void *__restrict__ c1, void *__restrict__ c2,
                                          const float *r0, const fk_gemm_params &p,
                                          const uint32_t *__restrict__ position = nullptr,
                                          const uint32_t *__restrict__ slot = nullptr,
                                          const float *__restrict__ rope = nullptr,
                                          const fk_gemm_rope_params &rp = fk_gemm_rope_params{}) {
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
#define FK_GEMM_LOAD_TILE(T, ST)                                                                          \
  do {                                                                                                    \
    const uint32_t so_ = (T) * TILEB;                                                                     \
    FK_LDS char *d_ = stage0 + (ST) * STAGEB;                                                             \
    _Pragma("unroll") for (int q = 0; q < 4; q++) {                                                       \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_src, d_ + q * 1024, 16, vl + q * 1024, so_, 0, 0);      \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_src, d_ + TILEB + q * 1024, 16, vl + q * 1024, so_, 0, 0); \
    }                                                                                                     \
  } while (0)

  // Fragment reads: lane l reads row l mod 32 of a 32-row block and logical
  // unit 2 h + l div 32 of the step's k-half h, at its swizzled place; A's
  // blocks are rows wm 128 + 32 i, B's columns wn 128 + 32 j of the tile, or
  // for SiLU·mul gate columns wn 64 + 32 j (blocks 0-1) and the same up
  // columns (blocks 2-3), so that a lane holds gate and up of one element.
  const uint32_t rsw = fk::tile_swizzle(lane % 16);
  const uint32_t ra = (wm * 128 + lane % 32) * ROW16;
  const uint32_t rb = TILEB / 16 + (wn * (MODE == FK_GEMM_SILU_MUL ? 64 : 128) + lane % 32) * ROW16;
  const uint32_t kc0 = (lane / 32) ^ rsw, kc1 = (2 + lane / 32) ^ rsw;
#define FK_GEMM_BROW(J) (MODE == FK_GEMM_SILU_MUL ? ((J) < 2 ? 32 * (J) : FK_GEMM_BN / 2 + 32 * ((J) - 2)) : 32 * (J))

  fk_float16v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  // Two sets of fragments: [A | B][k-half][block].
  fk::Half8 fr0[2][2][4], fr1[2][2][4];
#define FK_GEMM_READ(FA, FB, ST)                                                                          \
  do {                                                                                                    \
    const uint4 *s_ = gemm_lds + (ST) * (STAGEB / 16);                                                    \
    _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                       \
      FB[0][j].u = s_[rb + FK_GEMM_BROW(j) * ROW16 + kc0];                                                \
      FB[1][j].u = s_[rb + FK_GEMM_BROW(j) * ROW16 + kc1];                                                \
    }                                                                                                     \
    _Pragma("unroll") for (int i = 0; i < 4; i++) {                                                       \
      FA[0][i].u = s_[ra + 32 * i * ROW16 + kc0];                                                         \
      FA[1][i].u = s_[ra + 32 * i * ROW16 + kc1];                                                         \
    }                                                                                                     \
  } while (0)
  // The fragments stay in VGPRs: the matrix operation would also take them
  // from AGPRs, and an allocation that puts them there moves accumulators
  // around the loop.  The constraint also completes their reads here.
#define FK_GEMM_PIN(FA, FB)                                                                               \
  do {                                                                                                    \
    _Pragma("unroll") for (int h = 0; h < 2; h++)                                                         \
    _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                       \
      asm volatile("" : "+v"(FB[h][j].h));                                                                \
      asm volatile("" : "+v"(FA[h][j].h));                                                                \
    }                                                                                                     \
  } while (0)
#define FK_GEMM_MFMA(FA, FB)                                                                              \
  do {                                                                                                    \
    _Pragma("unroll") for (int h = 0; h < 2; h++)                                                         \
    _Pragma("unroll") for (int i = 0; i < 4; i++)                                                         \
    _Pragma("unroll") for (int j = 0; j < 4; j++)                                                         \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(FB[h][j].h, FA[h][i].h, acc[i][j], 0, 0, 0);     \
  } while (0)
  // s_waitcnt vmcnt(8), the other counters untouched: at most one tile's
  // loads (8 a thread) still in flight, so the one before it has landed.
#define FK_GEMM_WAIT_TILE() __builtin_amdgcn_s_waitcnt(8 | (0x7 << 4) | (0xf << 8))
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
  // One K step: tile s's fragments FC in registers, tile s + 1's read into
  // FN while FC is multiplied; the tile loads go out between the matrix
  // operations, one after every four.
#define FK_GEMM_STEP(FC, FN, T_LOAD, ST_LOAD, ST_READ)                                                   \
  do {                                                                                                    \
    FK_GEMM_WAIT_TILE();                                                                                  \
    FK_GEMM_BARRIER();                                                                                    \
    FK_GEMM_READ(FN[0], FN[1], ST_READ);                                                                  \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    FK_GEMM_MFMA(FC[0], FC[1]);                                                                           \
    FK_GEMM_LOAD_TILE(T_LOAD, ST_LOAD);                                                                   \
    _Pragma("unroll") for (int g_ = 0; g_ < 8; g_++) {                                                    \
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                                                  \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                                  \
    }                                                                                                     \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    FK_GEMM_PIN(FN[0], FN[1]);                                                                            \
  } while (0)

  // The pipeline.  At step s the fragments of tile s are in registers and
  // tiles s + 1, s + 2 are in LDS stages (s + 1) mod 4, (s + 2) mod 4 or on
  // their way there.  Step s waits for its own loads of tile s + 1, meets the
  // others at the barrier (after which all of tile s + 1 is in LDS), reads
  // tile s + 1's fragments, multiplies tile s's and loads tile s + 3 into
  // stage (s + 3) mod 4 (tile s - 1's, whose fragments every wave read before
  // this step's barrier).  Loads past the last tile repeat it into stages no
  // step reads.
  const uint32_t steps = k / FK_GEMM_BK;  // even
  const uint32_t last = steps - 1;
#define FK_GEMM_T(X) ((X) < last ? (X) : last)
  FK_GEMM_LOAD_TILE(0, 0);
  FK_GEMM_LOAD_TILE(FK_GEMM_T(1), 1);
  FK_GEMM_LOAD_TILE(FK_GEMM_T(2), 2);
  __builtin_amdgcn_s_waitcnt((1 << 14) | (0x7 << 4) | (0xf << 8));  // vmcnt(16): tile 0 landed
  FK_GEMM_BARRIER();
  FK_GEMM_READ(fr0[0], fr0[1], 0);
  FK_GEMM_PIN(fr0[0], fr0[1]);
  for (uint32_t s = 0; s < steps; s += 2) {
    FK_GEMM_STEP(fr0, fr1, FK_GEMM_T(s + 3), (s + 3) % FK_GEMM_STAGES, (s + 1) % FK_GEMM_STAGES);
    FK_GEMM_STEP(fr1, fr0, FK_GEMM_T(s + 4), (s + 4) % FK_GEMM_STAGES, (s + 2) % FK_GEMM_STAGES);
  }
  // Nothing may still be landing in LDS when the threadgroup ends.
  __builtin_amdgcn_s_waitcnt(0);
#undef FK_GEMM_LOAD_TILE
#undef FK_GEMM_READ
#undef FK_GEMM_PIN
#undef FK_GEMM_MFMA
#undef FK_GEMM_WAIT_TILE
#undef FK_GEMM_BARRIER
#undef FK_GEMM_STEP
#undef FK_GEMM_T
#undef FK_GEMM_BROW

  // Epilogue.  Block (i, j)'s lane l holds C row m = wm 128 + 32 i + l mod 32
  // and, for each g < 4, columns 32 j + 8 g + 4 (l div 32) .. + 3 (of the
  // wavefront's) as registers 4 g .. 4 g + 3.
  const uint32_t m = m0 + wm * 128 + lane % 32;
  const uint32_t nq = 4 * (lane / 32);
  if (MODE == FK_GEMM_SILU_MUL) {
    uint16_t *out = reinterpret_cast<uint16_t *>(c0);
    const uint32_t ncols = p.ldc[0];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          // Blocks 0-1: gate columns wn 64 + 32 j; blocks 2-3 the same up columns.
          const uint32_t n = n0 + wn * 64 + 32 * j + 8 * g + nq;
          uint16_t h[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float gt = acc[i][j][4 * g + r];
            const float u = acc[i][j + 2][4 * g + r];
            // silu(g) u = g / (1 + e^-g) · u with the hardware's exp and
            // reciprocal (a few ulp of binary32), then rounded once to f16
            // (2^-11): the f16 rounding bounds the error.  e^-g overflowing
            // gives silu 0, as the limit.
            const float e = __expf(-gt);
            h[r] = fk::to_f16(gt * __builtin_amdgcn_rcpf(1.0f + e) * u);
          }
          uint2 w;
          w.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
          w.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
          // Four consecutive columns of one row: half of one 16-byte unit.
          *reinterpret_cast<uint2 *>(out + fk::tile_offset(m + 32 * i, n, ncols)) = w;
        }
  } else if (MODE == FK_GEMM_QKV_ROPE) {
    // A 256-column tile is 4 whole heads; a lane's blocks 2 jp and 2 jp + 1
    // are the low and high halves of one head, so it holds both elements of
    // each pair RoPE turns (NeoX halves, as rope_elem: x_j c - x_{j+32} s below
    // the half, x_j c + x_{j-32} s above, the table's cos and sin of the row's
    // position).  q goes to f16 rows (the attention's), k and v to the caches
    // rounded as the decode step's stores round.
    const bool bf16 = rp.cache_bf16 != 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t row = m + 32 * i;
      const uint32_t pos = position[row];
      const uint32_t sl = min(slot[row], rp.slots - 1);
      const float *cs = rope + (size_t)min(pos, rp.rope_rows - 1) * 64;
#pragma unroll
      for (int jp = 0; jp < 2; jp++) {
        const uint32_t head = (n0 + wn * 128 + 64 * jp) / 64;
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const uint32_t d = 8 * g + nq;  // the low half's first of four columns; their partners d + 32 ..
          float lo[4], hi[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            lo[r] = acc[i][2 * jp][4 * g + r];
            hi[r] = acc[i][2 * jp + 1][4 * g + r];
          }
          if (anchor != 2) {
            const float4 t01 = *reinterpret_cast<const float4 *>(cs + 2 * d);      // (cos, sin) of pairs d, d + 1
            const float4 t23 = *reinterpret_cast<const float4 *>(cs + 2 * d + 4);  // pairs d + 2, d + 3
            const float cc[4] = {t01.x, t01.z, t23.x, t23.z};
            const float sn[4] = {t01.y, t01.w, t23.y, t23.w};
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const float x = lo[r] * cc[r] - hi[r] * sn[r];
              const float y = hi[r] * cc[r] + lo[r] * sn[r];
              lo[r] = x;
              hi[r] = y;
            }
          }
          if (anchor == 0) {
            uint16_t *q = reinterpret_cast<uint16_t *>(c0) + (size_t)row * p.ldc[0] + head * 64 + d;
            *reinterpret_cast<uint2 *>(q) = make_uint2(fk::to_f16(lo[0]) | ((uint32_t)fk::to_f16(lo[1]) << 16),
                                                       fk::to_f16(lo[2]) | ((uint32_t)fk::to_f16(lo[3]) << 16));
            *reinterpret_cast<uint2 *>(q + 32) = make_uint2(fk::to_f16(hi[0]) | ((uint32_t)fk::to_f16(hi[1]) << 16),
                                                            fk::to_f16(hi[2]) | ((uint32_t)fk::to_f16(hi[3]) << 16));
          } else {
            uint16_t *c = reinterpret_cast<uint16_t *>(anchor == 1 ? c1 : c2) +
                          (((size_t)sl * rp.kv_heads + head) * rp.length + pos % rp.length) * 64 + d;
            *reinterpret_cast<uint2 *>(c) =
                make_uint2(fk::narrow_cache(lo[0], bf16) | ((uint32_t)fk::narrow_cache(lo[1], bf16) << 16),
                           fk::narrow_cache(lo[2], bf16) | ((uint32_t)fk::narrow_cache(lo[3], bf16) << 16));
            *reinterpret_cast<uint2 *>(c + 32) =
                make_uint2(fk::narrow_cache(hi[0], bf16) | ((uint32_t)fk::narrow_cache(hi[1], bf16) << 16),
                           fk::narrow_cache(hi[2], bf16) | ((uint32_t)fk::narrow_cache(hi[3], bf16) << 16));
          }
        }
      }
    }
  } else {
    float *out = reinterpret_cast<float *>(anchor == 0 ? c0 : (anchor == 1 ? c1 : c2));
    const uint32_t ld = anchor == 0 ? p.ldc[0] : (anchor == 1 ? p.ldc[1] : p.ldc[2]);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const size_t at = (size_t)(m + 32 * i) * ld + n0 + wn * 128 + 32 * j + 8 * g + nq;
          fk_float4v v = fk_float4v{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          if (MODE == FK_GEMM_ADD) v = *reinterpret_cast<const fk_float4v *>(r0 + at) + v;
          *reinterpret_cast<fk_float4v *>(out + at) = v;
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
