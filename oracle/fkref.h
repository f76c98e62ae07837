/*
 * fkref.h — the oracle: a CPU restatement of FuryKernel's interpreter and CPU
 * target arithmetic (src/FuryKernel/Interp.hs, src/FuryKernel/Cpu.hs), of the
 * reference's reduction orders (src/FuryKernel/Reduce.hs, test/Test/FuryKernel/
 * Gemv.hs, test/Test/FuryKernel/Kernels.hs) and of the kernels of a planned
 * step, in plain C: lanes in lock-step, one thread, threadgroups in sequence
 * (src/FuryKernel/Cpu.hs:4-14,259-263).
 *
 * TEST INFRASTRUCTURE.  Only the tests, the smoke check and the benchmark's
 * CPU-baseline leg load this library, as the checker of the HIP kernels and
 * as the CPU baseline.  Nothing of the product links or calls it.
 *
 * Every reduction takes the SIMD width `width` as a parameter: 32 is the CPU
 * target's (src/FuryKernel/Cpu.hs:73), 64 is gfx950's wavefront.
 */
#ifndef FKREF_H
#define FKREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types, as the kernels' buffers hold them. */
enum { FKREF_F32 = 0, FKREF_F16 = 1, FKREF_BF16 = 2, FKREF_I8 = 3, FKREF_U32 = 4 };

/* Numerics (src/FuryKernel/Numerics.hs). */
float fkref_widen_bf16(uint16_t b);
uint16_t fkref_narrow_bf16(float x);
float fkref_widen_f16(uint16_t h);
uint16_t fkref_narrow_f16(float x);
uint16_t fkref_narrow_f16_f64(double x);
/* IEEE 754-2019 minimumNumber / maximumNumber as the interpreter has them
 * (src/FuryKernel/Interp.hs:940-956). */
float fkref_min(float a, float b);
float fkref_max(float a, float b);
/* rsqrt, exp, log, tanh: binary64's, rounded once to binary32
 * (src/FuryKernel/Interp.hs:828-854). */
float fkref_rsqrt(float x);
float fkref_exp(float x);

/* SIMD-group reductions: pairwise, neighbours first (src/FuryKernel/IR.hs:
 * 269-283, src/FuryKernel/Interp.hs:733-745). */
float fkref_simd_sum(const float *lanes, int width);
float fkref_simd_max(const float *lanes, int width);
/* Threadgroup reductions of one value per thread (src/FuryKernel/Reduce.hs:
 * 29-85): `threads` a multiple of `width`. */
float fkref_tg_reduce_sum(const float *per_thread, int threads, int width);
float fkref_tg_reduce_max(const float *per_thread, int threads, int width);
/* Split-K's combine: partials added in split order (src/FuryKernel/Reduce.hs:
 * 87-125). */
float fkref_combine_splits(const float *partials, int splits);

/* The GEMV of test/Test/FuryKernel/Gemv.hs:131-191, in its order.
 * W is [n, k] (out_in) of `wtype`, x is [m, k] of `xtype`, y is [m, n] f32.
 * pack: elements a lane loads at once (a multiple of 4); split: SIMD groups
 * sharing a row.  `row_scale` (n f32, or NULL) multiplies each output row's
 * sum: y = total * scale (the int8 weight-only layer). */
/* Threads the GEMVs' rows are spread over (1: the CPU target's one thread).
 * Each row's arithmetic is the same at any count. */
int fkref_set_threads(int threads);
int fkref_gemv(const void *w, int wtype, const void *x, int xtype, float *y, const float *row_scale, int n, int k,
               int m, int width, int pack, int split);

/* RMSNorm in the order of test/Test/FuryKernel/Kernels.hs:53-74, generalised
 * to packs and segments: one threadgroup of `threads` threads per segment;
 * thread t visits packs t, t + threads, ...; its sum of squares, then
 * tgReduceSum; scale = rsqrt(total / seg + eps); y = ((x * scale) * gamma) *
 * factor, gamma (seg f32) optional, factor skipped when 1. */
int fkref_rmsnorm(const float *x, const float *gamma, float *y, int rows, int width_elems, int seg, float eps,
                  float factor, int threads, int width, int pack);

/* A row softmax: tgReduceMax of the elements (from -inf), exp(x - max) in
 * binary64 rounded once, tgReduceSum of those (from -0), and each over the
 * sum (src/FuryKernel/Reduce.hs:39-47 for the reductions). */
int fkref_softmax(const float *x, float *y, int rows, int n, int threads, int width, int pack);

/* ------------------------------------------------------------------------ */
/* The kernels of a planned step, in the orders the gfx950 kernels compute
 * them (furykernel_amd/csrc/kernels/fk_step.h), their arithmetic the
 * evaluator's contract (src/FuryKernel/Program/Eval.hs:26-86).               */

/* Prologue and epilogue modes of a GEMV step. */
enum { FKREF_PRO_STORED = 0, FKREF_PRO_RMSNORM = 1, FKREF_PRO_GATHER = 2, FKREF_PRO_GATHER_RMSNORM = 3,
       FKREF_PRO_SILU_MUL = 4 };
enum { FKREF_EPI_NONE = 0, FKREF_EPI_ADD_STORED = 1, FKREF_EPI_ADD_GATHER = 2 };

/* A GEMV step: the anchors' input row made by the prologue (`threads`
 * threads for the RMSNorm's reduction), then each anchor's rows in the
 * reference GEMV's order at `width` (split 1, packs of 16 bytes), then the
 * epilogue.  `w[j]`/`y[j]` per anchor (y[j] NULL: not stored). */
int fkref_step_gemv(const void *const *w, int wtype, float *const *y, const int *rows, int n_anchors, int k,
                    int pro_mode, const float *src, const float *src2, const float *gamma, const void *table,
                    uint32_t token, int table_rows, int seg, float eps, float factor, float gfactor, int epi_mode,
                    const float *res, const void *res_table, uint32_t res_token, float *epi_out, int threads,
                    int width, int act, int src2_off);

/* RoPE (NeoX halves) of element j of a head of width d turned by `position`:
 * freq = theta^(-2i/d) and cos/sin in binary64 rounded once, the angle the
 * binary32 product position * freq. */
float fkref_rope_elem(const float *head, int j, int d, int rotated, uint32_t position, float theta);

/* KV stores of one row into ring caches (uint16 elements, f16 or bf16). */
int fkref_step_store(const float *x0, const float *x1, uint16_t *c0, uint16_t *c1, int n_stores, int rope0,
                     int rope1, int kv_heads, int head_dim, int length, int slots, int rotated, float theta,
                     uint32_t position, uint32_t slot, int cache_bf16);

/* Attention partials over splits of `split` (at most 128, a multiple of 8)
 * positions per KV head: partials[((h * splits + t) * (d + 2))] =
 * [max, sum, acc[d]]; the sums over 8 runs of split / 8 positions, each in
 * order of position, then the runs in order. */
int fkref_step_attend(const float *q, const uint16_t *kc, const uint16_t *vc, float *partials, int heads,
                      int kv_heads, int head_dim, int length, int slots, int splits, int split, int rope,
                      int rotated, float theta, float scale, int window, uint32_t position, uint32_t slot,
                      int cache_bf16);
int fkref_step_attend_reach(const float *q, const uint16_t *kc, const uint16_t *vc, float *partials, int heads,
                            int kv_heads, int head_dim, int length, int slots, int splits, int split, int rope,
                            int rotated, float theta, float scale, int window, uint32_t position, uint32_t slot,
                            uint32_t reach, int cache_bf16);
int fkref_step_attend_paged(const float *q, uint16_t *const *kp, uint16_t *const *vp, float *partials, int heads,
                            int kv_heads, int head_dim, int block_size, const uint32_t *table, int table_len,
                            int blocks, int splits, int split, int rope, int rotated, float theta, float scale,
                            int window, uint32_t position, uint32_t reach, int cache_bf16);
int fkref_step_store_paged(const float *x0, const float *x1, uint16_t *const *p0, uint16_t *const *p1,
                           int n_stores, int rope0, int rope1, int kv_heads, int head_dim, int block_size,
                           const uint32_t *table, int table_len, int blocks, int rotated, float theta,
                           uint32_t position, int cache_bf16);

/* The splits combined once, in split order. */
int fkref_step_attend_wide(const float *q, const uint16_t *kc, const uint16_t *vc, float *partials, int heads,
                           int kv_heads, int head_dim, int length, int slots, int splits, int split, int rope,
                           int rotated, float theta, float scale, int window, uint32_t position, uint32_t slot,
                           int cache_bf16);
int fkref_step_combine(const float *partials, float *out, int heads, int head_dim, int splits);

/* The index of the largest element, ties to the lowest (Eval.hs:681-685). */
uint32_t fkref_argmax(const float *x, int n);
/* The greedy token's fold as a maximum of 64-bit keys (the order of the value,
 * +0 and -0 equal, a NaN at index 0 above all and one elsewhere below all;
 * then the complement of the index): the key of one element, and the largest
 * key of a row of n (0 for n = 0). */
uint64_t fkref_argmax_key(float v, uint32_t index);
uint64_t fkref_argmax_keyed(const float *x, int n);
int fkref_route(const float *x, const float *scale, uint32_t *ids, float *ws, int n, int k, int has_scale);
int fkref_combine_ranks(const float *w, const float *x, const float *res, float *y, int seg, int ranks,
                        int residual);

/* SiLU(a) * b elementwise: a / (1 + exp(-a)) * b, exp binary64's rounded once. */
int fkref_silu_mul(const float *a, const float *b, float *y, int n);
/* The activations of an act·mul (FKREF_ACT_SILU, FKREF_ACT_GELU_TANH). */
enum { FKREF_ACT_SILU = 0, FKREF_ACT_GELU_TANH = 1 };
float fkref_tanh(float x);
float fkref_gelu_tanh(float a);
float fkref_softcap(float x, float cap);
int fkref_act_mul(const float *a, const float *b, float *y, int n, int act);

/* Element-wise forms of the numerics, for the IR interpreter (oracle/interp.py):
 * src/FuryKernel/Numerics.hs's conversions, IEEE 754's fusedMultiplyAdd of
 * binary32 (C's fmaf, one rounding), and rsqrt, exp, log and tanh of binary64
 * by the platform's libm, as the reference's interpreter computes them
 * (src/FuryKernel/Interp.hs:828-854). */
void fkref_widen_f16_n(const uint16_t *h, float *y, size_t n);
void fkref_widen_bf16_n(const uint16_t *b, float *y, size_t n);
void fkref_narrow_f16_n(const float *x, uint16_t *y, size_t n);
void fkref_narrow_bf16_n(const float *x, uint16_t *y, size_t n);
void fkref_narrow_f16_f64_n(const double *x, uint16_t *y, size_t n);
void fkref_fma_f32_n(const float *a, const float *b, const float *c, float *y, size_t n);
enum { FKREF_RSQRT = 0, FKREF_EXP = 1, FKREF_LOG = 2, FKREF_TANH = 3 };
void fkref_unary_f64_n(int op, const double *x, double *y, size_t n);

#ifdef __cplusplus
}
#endif

#endif /* FKREF_H */
