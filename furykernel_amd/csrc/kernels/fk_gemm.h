// fk_gemm.h — the prefill GEMM: C = A · Bᵀ on the matrix cores (gfx950 MFMA),
// the Linear anchors of a step of many rows (src/FuryKernel/Tile.hs:76-157:
// C = A·Bᵀ tiles staged in threadgroup memory; here f16 operands, binary32
// accumulation).
//
// Layout in HBM: A is [M, K] f16 row-major (the step's input rows, rounded
// once to f16), B is [N, K] f16 row-major (the `out_in` weights), both
// K-contiguous; C is [M, ldc] f32 (or f16 for the SiLU·mul epilogue).
//
// A threadgroup of 4 wavefronts (one a SIMD, each with the whole register
// file's share of 512) takes a 256 × 256 tile of C (for the SiLU·mul epilogue,
// 256 rows × 128 columns of gate and the same 128 of up).  Each K step of 32 is
// staged in LDS, rows padded to 40 halves (80 bytes) so that the 16 lanes
// reading 16 bytes of 16 different rows start at 16 distinct bank groups; the
// next step's tile is loaded into registers while the current one is
// multiplied.  Wavefront
// (wm, wn) holds 128 × 128 of the tile as 8 × 8 blocks of 16 × 16, each
// accumulated by v_mfma_f32_16x16x32_f16: 64 matrix operations a wavefront for
// each K step, on 16 16-byte operand loads from LDS.
//
// v_mfma_f32_16x16x32_f16 (D = A B + C, A 16 × 32, B 32 × 16): lane l holds
// A[l mod 16][8 (l div 16) .. + 7] and B[8 (l div 16) .. + 7][l mod 16] as 8
// halves each, and D[4 (l div 16) .. + 3][l mod 16] as 4 floats.
//
// The order of the sums over k is the matrix core's; results are held to the
// binary32 accumulation bound of the f16 products (the contract of Tile.hs's
// fragments), not to bits.
#pragma once

#include "fk_common.h"

#define FK_GEMM_THREADS 256
#define FK_GEMM_BM 256
#define FK_GEMM_BN 256
#define FK_GEMM_BK 32
#define FK_GEMM_LDSROW 40  // halves a staged row takes: 32 and 8 of padding

typedef _Float16 fk_half8 __attribute__((ext_vector_type(8)));
typedef float fk_float4v __attribute__((ext_vector_type(4)));

enum : uint32_t {
  FK_GEMM_STORE = 0,     // C = A Bᵀ (f32)
  FK_GEMM_ADD = 1,       // C = R + A Bᵀ (f32), R [M, ldc]
  FK_GEMM_SILU_MUL = 2,  // C = f16(silu(A B0ᵀ) · (A B1ᵀ)) (f16): gate B0, up B1
};

struct fk_gemm_params {
  uint32_t m;            // rows of A and C, a multiple of 256
  uint32_t k;            // a multiple of 32
  uint32_t n_anchors;    // 1 to 3 weights (SiLU·mul: 2, gate and up)
  uint32_t first_col[4]; // anchor j's columns of C are [first_col[j], first_col[j + 1]), each a multiple of 256
  uint32_t ldc[3];       // row stride of anchor j's output (its columns)
};

namespace fk {

union Half8 {
  fk_half8 h;
  uint4 u;
};

}  // namespace fk

// One threadgroup's tile.  MODE: the epilogue.
template <uint32_t MODE>
__device__ __forceinline__ void gemm_tile(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0,
                                          const _Float16 *__restrict__ b1, const _Float16 *__restrict__ b2,
                                          void *__restrict__ c0, void *__restrict__ c1, void *__restrict__ c2,
                                          const float *__restrict__ r0, const fk_gemm_params &p) {
  extern __shared__ uint4 gemm_lds[];
  uint4 *as = gemm_lds;                                        // [256][40 halves]
  uint4 *bs = gemm_lds + FK_GEMM_BM * FK_GEMM_LDSROW / 8;      // [256][40 halves]
  constexpr uint32_t ROW16 = FK_GEMM_LDSROW / 8;               // 16-byte units a staged row takes
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

  // Which weights the tile's 256 B rows come from: a plain tile's columns
  // [n0, n0 + 256) of one anchor; a SiLU·mul tile's gate rows [n0, n0 + 128)
  // then up rows [n0, n0 + 128).
  const _Float16 *bt0;
  const _Float16 *bt1;
  uint32_t anchor = 0, n0 = 0;
  if (MODE == FK_GEMM_SILU_MUL) {
    n0 = tn * (FK_GEMM_BN / 2);
    bt0 = b0 + (size_t)n0 * k;
    bt1 = b1 + (size_t)n0 * k;
  } else {
    const uint32_t col = tn * FK_GEMM_BN;
    anchor = (p.n_anchors > 1 && col >= p.first_col[1] ? 1u : 0u) + (p.n_anchors > 2 && col >= p.first_col[2] ? 1u : 0u);
    n0 = col - (anchor == 0 ? p.first_col[0] : (anchor == 1 ? p.first_col[1] : p.first_col[2]));
    const _Float16 *bw = anchor == 0 ? b0 : (anchor == 1 ? b1 : b2);
    bt0 = bw + (size_t)n0 * k;
    bt1 = bt0 + (size_t)(FK_GEMM_BN / 2) * k;
  }

  // Global loads of a K step: thread t takes 16-byte chunk t mod 4 of rows
  // t div 4 + 64 i (i < 4) of A's tile and of B's (the B tile's first 128
  // rows from bt0, the last 128 from bt1).
  const uint32_t lr = tid / 4;
  const uint32_t lc = tid % 4;
  // Row i of the thread's: A row m0 + lr + 64 i; B row lr + 64 i of the tile.
  const _Float16 *ap = a + (size_t)(m0 + lr) * k + 8 * lc;
  const _Float16 *bp0 = bt0 + (size_t)lr * k + 8 * lc;  // rows lr, lr + 64 (the tile's first half)
  const _Float16 *bp1 = bt1 + (size_t)lr * k + 8 * lc;  // rows lr + 128, lr + 192
  const size_t step64 = (size_t)64 * k;
  uint4 ga0, ga1, ga2, ga3, gb0, gb1, gb2, gb3;
#define FK_GEMM_LOAD(K0)                                                       \
  do {                                                                         \
    ga0 = *reinterpret_cast<const uint4 *>(ap + (K0));                         \
    ga1 = *reinterpret_cast<const uint4 *>(ap + step64 + (K0));                \
    ga2 = *reinterpret_cast<const uint4 *>(ap + 2 * step64 + (K0));            \
    ga3 = *reinterpret_cast<const uint4 *>(ap + 3 * step64 + (K0));            \
    gb0 = *reinterpret_cast<const uint4 *>(bp0 + (K0));                        \
    gb1 = *reinterpret_cast<const uint4 *>(bp0 + step64 + (K0));               \
    gb2 = *reinterpret_cast<const uint4 *>(bp1 + (K0));                        \
    gb3 = *reinterpret_cast<const uint4 *>(bp1 + step64 + (K0));               \
  } while (0)
#define FK_GEMM_STAGE()                                                        \
  do {                                                                         \
    as[lr * ROW16 + lc] = ga0;                                                 \
    as[(lr + 64) * ROW16 + lc] = ga1;                                          \
    as[(lr + 128) * ROW16 + lc] = ga2;                                         \
    as[(lr + 192) * ROW16 + lc] = ga3;                                         \
    bs[lr * ROW16 + lc] = gb0;                                                 \
    bs[(lr + 64) * ROW16 + lc] = gb1;                                          \
    bs[(lr + 128) * ROW16 + lc] = gb2;                                         \
    bs[(lr + 192) * ROW16 + lc] = gb3;                                         \
  } while (0)

  // The wavefront's B rows of the staged tile: 8 blocks of 16; for SiLU·mul,
  // gate columns wn 64 .. + 63 (blocks 0-3) and the same up columns (blocks
  // 4-7), so a lane holds gate and up of one element together.
  uint32_t brow0[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    if (MODE == FK_GEMM_SILU_MUL)
      brow0[j] = (j < 4 ? wn * 64 + 16 * j : FK_GEMM_BN / 2 + wn * 64 + 16 * (j - 4));
    else
      brow0[j] = wn * 128 + 16 * j;
  }

  fk_float4v acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[i][j] = fk_float4v{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t steps = k / FK_GEMM_BK;
  FK_GEMM_LOAD(0);
  FK_GEMM_STAGE();
  __syncthreads();
  for (uint32_t s = 0; s < steps; s++) {
    if (s + 1 < steps) FK_GEMM_LOAD((s + 1) * FK_GEMM_BK);
#pragma unroll
    for (int kk = 0; kk < FK_GEMM_BK / 32; kk++) {
      const uint32_t kc = kk * 4 + lane / 16;  // 16-byte unit of the staged row: k = 32 kk + 8 (l div 16)
      fk::Half8 fa[8], fb[8];
#pragma unroll
      for (int i = 0; i < 8; i++) fa[i].u = as[(wm * 128 + 16 * i + lane % 16) * ROW16 + kc];
#pragma unroll
      for (int j = 0; j < 8; j++) fb[j].u = bs[(brow0[j] + lane % 16) * ROW16 + kc];
#pragma unroll
      for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i].h, fb[j].h, acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (s + 1 < steps) {
      FK_GEMM_STAGE();
      __syncthreads();
    }
  }
#undef FK_GEMM_LOAD
#undef FK_GEMM_STAGE

  // Epilogue: lane l holds rows 4 (l div 16) .. + 3 of each 16 × 16 block, column l mod 16.
  const uint32_t col_in = lane % 16;
  const uint32_t row_in = 4 * (lane / 16);
  if (MODE == FK_GEMM_SILU_MUL) {
    uint16_t *out = reinterpret_cast<uint16_t *>(c0);
    const uint32_t ld = p.ldc[0];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          // Blocks 0-3: gate columns wn 64 + 16 j; blocks 4-7 the same up columns.
          const uint32_t m = m0 + wm * 128 + 16 * i + row_in + r;
          const uint32_t n = n0 + wn * 64 + 16 * j + col_in;
          const float g = acc[i][j][r];
          const float u = acc[i][j + 4][r];
          // e^-g by the device library's binary32 exp (within the 4 ulp the
          // evaluator's contract allows, src/FuryKernel/Program/Eval.hs:48):
          // binary64's here would spill the accumulators.
          const float e = expf(-g);
          out[(size_t)m * ld + n] = fk::narrow_f16((g / (1.0f + e)) * u);
        }
  } else {
    float *out = reinterpret_cast<float *>(anchor == 0 ? c0 : (anchor == 1 ? c1 : c2));
    const uint32_t ld = anchor == 0 ? p.ldc[0] : (anchor == 1 ? p.ldc[1] : p.ldc[2]);
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t m = m0 + wm * 128 + 16 * i + row_in + r;
          const uint32_t n = n0 + wn * 128 + 16 * j + col_in;
          const size_t at = (size_t)m * ld + n;
          const float v = acc[i][j][r];
          out[at] = MODE == FK_GEMM_ADD ? r0[at] + v : v;
        }
  }
}

// Buffers in binding order, then the parameter struct.  The grid: one
// threadgroup a tile, tiles of 256 rows down M first.
#define FK_GEMM_ENTRY(NAME, MODE)                                                                                   \
  extern "C" __global__ void __launch_bounds__(FK_GEMM_THREADS)                                                     \
      NAME(const _Float16 *__restrict__ a, const _Float16 *__restrict__ b0, const _Float16 *__restrict__ b1,      \
           const _Float16 *__restrict__ b2, void *__restrict__ c0, void *__restrict__ c1, void *__restrict__ c2,   \
           const float *__restrict__ r0, fk_gemm_params p) {                                                       \
    gemm_tile<MODE>(a, b0, b1, b2, c0, c1, c2, r0, p);                                                            \
  }

FK_GEMM_ENTRY(fk_gemm_f16_store, FK_GEMM_STORE)
FK_GEMM_ENTRY(fk_gemm_f16_add, FK_GEMM_ADD)
FK_GEMM_ENTRY(fk_gemm_f16_silu_mul, FK_GEMM_SILU_MUL)
