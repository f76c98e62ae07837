/*
 * fkref.c — the oracle's C restatement (see fkref.h).
 *
 * TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this, as the checker and the CPU baseline.
 *
 * Built with -O2 -ffp-contract=off and no fast-math, so each C operation on
 * floats is one IEEE 754 operation rounded once, as the CPU target's Rust is
 * (src/FuryKernel/Backend.hs:52-73: Strict, no contraction).
 */
#include "fkref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Numerics: src/FuryKernel/Numerics.hs                                      */

static uint32_t bits_of(float x) {
  uint32_t w;
  memcpy(&w, &x, 4);
  return w;
}

static float float_of(uint32_t w) {
  float x;
  memcpy(&x, &w, 4);
  return x;
}

/* widenBF16 (Numerics.hs:33-39): the upper half of a binary32; NaN quiet. */
float fkref_widen_bf16(uint16_t b) {
  uint32_t w = (uint32_t)b << 16;
  if ((w & 0x7F800000u) == 0x7F800000u && (w & 0x007FFFFFu) != 0) w |= 0x00400000u;
  return float_of(w);
}

/* narrowBF16 (Numerics.hs:41-49): RNE by adding 0x7FFF plus the kept lsb. */
uint16_t fkref_narrow_bf16(float x) {
  uint32_t w = bits_of(x);
  if (isnan(x)) return (uint16_t)((w >> 16) | 0x0040);
  uint32_t lsb = (w >> 16) & 1u;
  return (uint16_t)((w + 0x7FFFu + lsb) >> 16);
}

/* widenF16 (Numerics.hs:51-71): exact, subnormals normalised, NaN quiet. */
float fkref_widen_f16(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t mag;
  if (e == 0x1F && m != 0) {
    mag = 0x7FC00000u | (m << 13);
  } else if (e == 0x1F) {
    mag = 0x7F800000u;
  } else if (e != 0) {
    mag = ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    mag = 0;
  } else {
    int shift = 0; /* leading zeros of the 10-bit mantissa */
    while (!(m & (0x200u >> shift))) shift++;
    uint32_t m2 = (m << (shift + 1)) & 0x3FFu;
    mag = ((uint32_t)(113 - shift - 1) << 23) | (m2 << 13);
  }
  return float_of(sign | mag);
}

/* roundShifted (Numerics.hs:159-167). */
static uint64_t round_shifted(uint64_t kept, uint64_t dropped, int width) {
  uint64_t half = (uint64_t)1 << (width - 1);
  if (dropped > half || (dropped == half && (kept & 1u))) return kept + 1;
  return kept;
}

/* narrowF16 (Numerics.hs:100-130): RNE with gradual underflow. */
uint16_t fkref_narrow_f16(float x) {
  uint32_t w = bits_of(x);
  uint16_t sign = (uint16_t)((w >> 16) & 0x8000u);
  int e = (int)((w >> 23) & 0xFFu);
  uint32_t m = w & 0x7FFFFFu;
  int unbiased = e - 127;
  uint16_t mag;
  if (e == 0xFF && m != 0) {
    mag = (uint16_t)(0x7E00u | (m >> 13));
  } else if (e == 0xFF) {
    mag = 0x7C00;
  } else if (unbiased >= 16) {
    mag = 0x7C00;
  } else if (unbiased >= -14) {
    uint32_t r = ((uint32_t)(unbiased + 15) << 10) | (m >> 13);
    mag = (uint16_t)round_shifted(r, m & 0x1FFFu, 13);
  } else {
    int shift = -(unbiased + 1);
    uint32_t full = m | 0x800000u;
    if (shift > 24) {
      mag = 0;
    } else {
      mag = (uint16_t)round_shifted(full >> shift, full & ((1u << shift) - 1u), shift);
    }
  }
  return (uint16_t)(sign | mag);
}

/* narrowF16Double (Numerics.hs:132-157): binary64 to binary16 in one rounding. */
uint16_t fkref_narrow_f16_f64(double x) {
  uint64_t w;
  memcpy(&w, &x, 8);
  uint16_t sign = (uint16_t)((w >> 48) & 0x8000u);
  int e = (int)((w >> 52) & 0x7FFu);
  uint64_t m = w & 0xFFFFFFFFFFFFFull;
  int unbiased = e - 1023;
  uint16_t mag;
  if (e == 0x7FF && m != 0) {
    mag = (uint16_t)(0x7E00u | (uint16_t)(m >> 42));
  } else if (e == 0x7FF) {
    mag = 0x7C00;
  } else if (unbiased >= 16) {
    mag = 0x7C00;
  } else if (unbiased >= -14) {
    uint64_t r = ((uint64_t)(unbiased + 15) << 10) | (m >> 42);
    mag = (uint16_t)round_shifted(r, m & ((1ull << 42) - 1), 42);
  } else {
    int shift = 28 - unbiased;
    uint64_t full = m | (1ull << 52);
    if (shift > 53) {
      mag = 0;
    } else {
      mag = (uint16_t)round_shifted(full >> shift, full & ((1ull << shift) - 1), shift);
    }
  }
  return (uint16_t)(sign | mag);
}

/* minimumNumber / maximumNumber (Interp.hs:940-956). */
float fkref_min(float x, float y) {
  if (isnan(x)) return isnan(y) ? float_of(0x7FC00000u) : y;
  if (isnan(y) || x < y) return x;
  if (y < x) return y;
  return float_of(bits_of(x) | bits_of(y));
}

float fkref_max(float x, float y) {
  if (isnan(x)) return isnan(y) ? float_of(0x7FC00000u) : y;
  if (isnan(y) || x > y) return x;
  if (y > x) return y;
  return float_of(bits_of(x) & bits_of(y));
}

/* Transcendentals in binary64, rounded once (Interp.hs:828-854). */
float fkref_rsqrt(float x) { return (float)(1.0 / sqrt((double)x)); }

float fkref_exp(float x) { return (float)exp((double)x); }
float fkref_tanh(float x) { return (float)tanh((double)x); }

/* GELU in its tanh form (src/FuryKernel/Program/Eval.hs:658-659) in binary32,
 * left to right as the formula reads, its constants rounded once and tanh
 * binary64's rounded once: (0.5 a) (1 + tanh(c0 (a + ((c1 a) a) a))). */
float fkref_gelu_tanh(float a) {
  const float c0 = 0.7978845608028654f; /* sqrt(2 / pi) */
  const float c1 = 0.044715f;
  float cube = ((c1 * a) * a) * a;
  float t = fkref_tanh(c0 * (a + cube));
  return (0.5f * a) * (1.0f + t);
}

/* A softcap (Eval.hs:384-390): cap tanh(x / cap). */
float fkref_softcap(float x, float cap) { return cap * fkref_tanh(x / cap); }

/* ------------------------------------------------------------------------ */
/* Reductions: Interp.hs:733-745, Reduce.hs                                  */

/* Pairwise, neighbours first: ((x0+x1)+(x2+x3))+...; an odd lane out goes on
 * as it is (Interp.hs:733-745).  width <= 1024. */
static float simd_reduce(const float *lanes, int width, int is_max) {
  float buf[1024];
  int n = width;
  if (n <= 0) return is_max ? -INFINITY : -0.0f;
  memcpy(buf, lanes, sizeof(float) * (size_t)n);
  while (n > 1) {
    int out = 0;
    int i = 0;
    for (; i + 1 < n; i += 2) buf[out++] = is_max ? fkref_max(buf[i], buf[i + 1]) : buf[i] + buf[i + 1];
    if (i < n) buf[out++] = buf[i];
    n = out;
  }
  return buf[0];
}

float fkref_simd_sum(const float *lanes, int width) { return simd_reduce(lanes, width, 0); }

float fkref_simd_max(const float *lanes, int width) { return simd_reduce(lanes, width, 1); }

/* tgReduce (Reduce.hs:55-85): each SIMD group's reduction in its slot; the
 * first group's lane l folds slots l, l + width, ... from the neutral value;
 * then one more SIMD reduction. */
static float tg_reduce(const float *v, int threads, int width, int is_max) {
  int groups = threads / width;
  float slots[1024];
  float lanes[1024];
  for (int g = 0; g < groups; g++) slots[g] = simd_reduce(v + (size_t)g * width, width, is_max);
  for (int l = 0; l < width; l++) {
    float acc = is_max ? -INFINITY : -0.0f;
    for (int k = l; k < groups; k += width) acc = is_max ? fkref_max(acc, slots[k]) : acc + slots[k];
    lanes[l] = acc;
  }
  return simd_reduce(lanes, width, is_max);
}

float fkref_tg_reduce_sum(const float *v, int threads, int width) { return tg_reduce(v, threads, width, 0); }

float fkref_tg_reduce_max(const float *v, int threads, int width) { return tg_reduce(v, threads, width, 1); }

/* combineSplits (Reduce.hs:112-125): ((p0 + p1) + p2) + ... */
float fkref_combine_splits(const float *p, int splits) {
  float acc = p[0];
  for (int q = 1; q < splits; q++) acc = acc + p[q];
  return acc;
}

/* ------------------------------------------------------------------------ */
/* GEMV: test/Test/FuryKernel/Gemv.hs:131-191                                */

static float element(const void *base, int type, size_t i) {
  switch (type) {
    case FKREF_F32: return ((const float *)base)[i];
    case FKREF_F16: return fkref_widen_f16(((const uint16_t *)base)[i]);
    case FKREF_BF16: return fkref_widen_bf16(((const uint16_t *)base)[i]);
    case FKREF_I8: return (float)((const int8_t *)base)[i];
    default: return NAN;
  }
}

/* Threads the GEMV's rows are spread over (the CPU target runs threadgroups
 * one after another on one thread; the all-cores figure spreads them, with
 * every row's arithmetic unchanged). */
static int g_threads = 1;

int fkref_set_threads(int threads) {
  if (threads < 1 || threads > 1024) return -1;
  g_threads = threads;
  return 0;
}

/* Row j of input row i, in the reference GEMV's order. */
static float gemv_row(const void *w, int wtype, const void *x, int xtype, int i, int j, int k, int width, int pack,
                      int split) {
  const int packs = k / pack;
  const int vlanes = split * width;
  const int chains = pack / 4;
  float small[4096];
  float *lane_total = vlanes <= 4096 ? small : (float *)malloc(sizeof(float) * (size_t)vlanes);
  float acc[16];
  float partial[64];
  if (!lane_total) return __builtin_nanf("");
  for (int v = 0; v < vlanes; v++) {
    /* Lane v of the virtual lanes (split q = v / width) visits packs
     * v, v + split * width, ...; each pack's elements go four to a chain,
     * ((x0 w0 + x1 w1) + (x2 w2 + x3 w3)), each chain its own sum. */
    for (int c = 0; c < chains; c++) acc[c] = 0.0f;
    for (int jp = v; jp < packs; jp += vlanes) {
      for (int c = 0; c < chains; c++) {
        size_t at = (size_t)jp * pack + 4 * c;
        float p0 = element(x, xtype, (size_t)i * k + at) * element(w, wtype, (size_t)j * k + at);
        float p1 = element(x, xtype, (size_t)i * k + at + 1) * element(w, wtype, (size_t)j * k + at + 1);
        float p2 = element(x, xtype, (size_t)i * k + at + 2) * element(w, wtype, (size_t)j * k + at + 2);
        float p3 = element(x, xtype, (size_t)i * k + at + 3) * element(w, wtype, (size_t)j * k + at + 3);
        acc[c] = acc[c] + ((p0 + p1) + (p2 + p3));
      }
    }
    /* The lane's chains in order (Gemv.hs:216-220, inOrder). */
    float t = acc[0];
    for (int c = 1; c < chains; c++) t = t + acc[c];
    lane_total[v] = t;
  }
  for (int q = 0; q < split; q++) partial[q] = fkref_simd_sum(lane_total + (size_t)q * width, width);
  if (lane_total != small) free(lane_total);
  return fkref_combine_splits(partial, split);
}

int fkref_gemv(const void *w, int wtype, const void *x, int xtype, float *y, const float *row_scale, int n, int k,
               int m, int width, int pack, int split) {
  if (n < 0 || k <= 0 || m <= 0 || width <= 0 || width > 1024 || pack < 4 || pack > 64 || pack % 4 || k % pack ||
      split <= 0 || split > 64)
    return -1;
  for (int i = 0; i < m; i++) {
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (int j = 0; j < n; j++) {
      float total = gemv_row(w, wtype, x, xtype, i, j, k, width, pack, split);
      if (row_scale) total = total * row_scale[j];
      y[(size_t)i * n + j] = total;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* RMSNorm: test/Test/FuryKernel/Kernels.hs:53-74                            */

int fkref_rmsnorm(const float *x, const float *gamma, float *y, int rows, int width_elems, int seg, float eps,
                  float factor, int threads, int width, int pack) {
  if (rows < 0 || seg <= 0 || width_elems % seg || seg % pack || threads % width || threads > 1024) return -1;
  float acc[1024];
  const int segs = width_elems / seg;
  const int packs = seg / pack;
  for (int r = 0; r < rows; r++) {
    for (int s = 0; s < segs; s++) {
      const float *xs = x + (size_t)r * width_elems + (size_t)s * seg;
      float *ys = y + (size_t)r * width_elems + (size_t)s * seg;
      for (int t = 0; t < threads; t++) {
        float a = 0.0f;
        for (int j = t; j < packs; j += threads) {
          for (int e = 0; e < pack; e++) {
            float v = xs[(size_t)j * pack + e];
            a = a + v * v;
          }
        }
        acc[t] = a;
      }
      float total = fkref_tg_reduce_sum(acc, threads, width);
      float scale = fkref_rsqrt(total / (float)seg + eps);
      for (int i = 0; i < seg; i++) {
        float v = xs[i] * scale;
        if (gamma) v = v * gamma[i];
        if (factor != 1.0f) v = v * factor;
        ys[i] = v;
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Row softmax (the reductions of src/FuryKernel/Reduce.hs:29-85)            */

int fkref_softmax(const float *x, float *y, int rows, int n, int threads, int width, int pack) {
  if (rows < 0 || n <= 0 || n % pack || threads % width || threads > 1024) return -1;
  float acc[1024];
  const int packs = n / pack;
  for (int r = 0; r < rows; r++) {
    const float *xs = x + (size_t)r * n;
    float *ys = y + (size_t)r * n;
    for (int t = 0; t < threads; t++) {
      float a = -INFINITY;
      for (int j = t; j < packs; j += threads)
        for (int e = 0; e < pack; e++) a = fkref_max(a, xs[(size_t)j * pack + e]);
      acc[t] = a;
    }
    float top = fkref_tg_reduce_max(acc, threads, width);
    for (int t = 0; t < threads; t++) {
      float a = -0.0f;
      for (int j = t; j < packs; j += threads)
        for (int e = 0; e < pack; e++) a = a + fkref_exp(xs[(size_t)j * pack + e] - top);
      acc[t] = a;
    }
    float total = fkref_tg_reduce_sum(acc, threads, width);
    for (int i = 0; i < n; i++) ys[i] = fkref_exp(xs[i] - top) / total;
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* The kernels of a planned step                                             */

static float silu_mul_1(float a, float b) {
  float e = fkref_exp(-a);
  float d = 1.0f + e;
  return (a / d) * b;
}

static float act_mul_1(float a, float b, int act) {
  return act == FKREF_ACT_GELU_TANH ? fkref_gelu_tanh(a) * b : silu_mul_1(a, b);
}

int fkref_act_mul(const float *a, const float *b, float *y, int n, int act) {
  if (act != FKREF_ACT_SILU && act != FKREF_ACT_GELU_TANH) return -1;
  for (int i = 0; i < n; i++) y[i] = act_mul_1(a[i], b[i], act);
  return 0;
}

int fkref_silu_mul(const float *a, const float *b, float *y, int n) {
  for (int i = 0; i < n; i++) y[i] = silu_mul_1(a[i], b[i]);
  return 0;
}

static size_t elem_bytes(int type) {
  switch (type) {
    case FKREF_F32: return 4;
    case FKREF_F16:
    case FKREF_BF16: return 2;
    case FKREF_I8: return 1;
    default: return 0;
  }
}

int fkref_step_gemv(const void *const *w, int wtype, float *const *y, const int *rows, int n_anchors, int k,
                    int pro_mode, const float *src, const float *src2, const float *gamma, const void *table,
                    uint32_t token, int table_rows, int seg, float eps, float factor, float gfactor, int epi_mode,
                    const float *res, const void *res_table, uint32_t res_token, float *epi_out, int threads,
                    int width, int act, int src2_off) {
  if (n_anchors < 1 || n_anchors > 3 || k <= 0) return -1;
  float *x = (float *)malloc(sizeof(float) * (size_t)k);
  if (!x) return -2;
  uint32_t tok = token < (uint32_t)table_rows ? token : (uint32_t)(table_rows - 1);
  for (int i = 0; i < k; i++) {
    switch (pro_mode) {
      case FKREF_PRO_GATHER:
      case FKREF_PRO_GATHER_RMSNORM: x[i] = element(table, wtype, (size_t)tok * k + i) * gfactor; break;
      case FKREF_PRO_SILU_MUL: x[i] = act_mul_1(src[i], src2[src2_off + i], act); break;
      default: x[i] = src[i]; break;
    }
  }
  if (pro_mode == FKREF_PRO_RMSNORM || pro_mode == FKREF_PRO_GATHER_RMSNORM) {
    int st = fkref_rmsnorm(x, gamma, x, 1, k, seg, eps, factor, threads, width, 4);
    if (st) {
      free(x);
      return st;
    }
  }
  const int pack = (int)(16 / elem_bytes(wtype));
  uint32_t rtok = res_token < (uint32_t)table_rows ? res_token : (uint32_t)(table_rows - 1);
  for (int a = 0; a < n_anchors; a++) {
    const int n = rows[a];
    float *t = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    if (!t) {
      free(x);
      return -2;
    }
    int st = fkref_gemv(w[a], wtype, x, FKREF_F32, t, NULL, n, k, 1, width, pack, 1);
    if (st) {
      free(t);
      free(x);
      return st;
    }
    for (int r = 0; r < n; r++) {
      if (y[a]) y[a][r] = t[r];
      if (epi_mode == FKREF_EPI_ADD_STORED) epi_out[r] = res[r] + t[r];
      if (epi_mode == FKREF_EPI_ADD_GATHER) epi_out[r] = element(res_table, wtype, (size_t)rtok * n + r) * gfactor + t[r];
    }
    free(t);
  }
  free(x);
  return 0;
}

float fkref_rope_elem(const float *head, int j, int d, int rotated, uint32_t position, float theta) {
  int half = d / 2;
  int i = j < half ? j : j - half;
  if (i >= rotated) return head[j];
  float freq = (float)pow((double)theta, -(double)(2 * i) / (double)d);
  float angle = (float)position * freq;
  float c = (float)cos((double)angle);
  float s = (float)sin((double)angle);
  return j < half ? head[j] * c - head[j + half] * s : head[j] * c + head[j - half] * s;
}

static uint16_t narrow_cache(float v, int bf16) { return bf16 ? fkref_narrow_bf16(v) : fkref_narrow_f16(v); }

static float widen_cache(uint16_t h, int bf16) { return bf16 ? fkref_widen_bf16(h) : fkref_widen_f16(h); }

/* Where a cached row (position t, kv head h) starts.  A ring (Graph.hs:
 * 138-143): slot s's ring of `length` positions, ((s kvHeads + h) length + t
 * mod length) headDim.  A paged pool (Graph.hs:144-152): block table[t /
 * blockSize] of the row's block table, (h blockSize + t mod blockSize)
 * headDim within it, the blocks anywhere (an array of their addresses).
 * Indexes past the table or the pool are clamped into them, as the kernels
 * clamp them (the gate keeps a valid program's inside). */
typedef struct {
  int paged;
  int kv_heads, head_dim;
  int length; uint32_t slot;                                  /* a ring */
  int block_size, table_len, blocks; const uint32_t *table;   /* a pool */
} fkref_rows;

static size_t row_index(const fkref_rows *L, uint32_t t, int h, uint32_t *block) {
  if (!L->paged) {
    *block = 0;
    return (((size_t)L->slot * L->kv_heads + h) * L->length + t % (uint32_t)L->length) * L->head_dim;
  }
  uint32_t ti = t / (uint32_t)L->block_size;
  if (ti >= (uint32_t)L->table_len) ti = (uint32_t)L->table_len - 1;
  uint32_t b = L->table[ti];
  *block = b < (uint32_t)L->blocks ? b : (uint32_t)L->blocks - 1;
  return ((size_t)h * L->block_size + t % (uint32_t)L->block_size) * L->head_dim;
}

/* A cache's row: `cache` for a ring, `pool[block]` for a paged pool. */
static uint16_t *row_of(const fkref_rows *L, uint16_t *cache, uint16_t *const *pool, uint32_t t, int h) {
  uint32_t b;
  size_t at = row_index(L, t, h, &b);
  return (L->paged ? pool[b] : cache) + at;
}

static int store_rows(const fkref_rows *L, const float *x0, const float *x1, uint16_t *c0, uint16_t *c1,
                      uint16_t *const *p0, uint16_t *const *p1, int n_stores, int rope0, int rope1, int rotated,
                      float theta, uint32_t position, int cache_bf16) {
  const int head_dim = L->head_dim;
  const int width = L->kv_heads * head_dim;
  for (int st = 0; st < n_stores; st++) {
    const float *x = st == 0 ? x0 : x1;
    int rope = st == 0 ? rope0 : rope1;
    for (int e = 0; e < width; e++) {
      int h = e / head_dim;
      int i = e % head_dim;
      float v = rope ? fkref_rope_elem(x + (size_t)h * head_dim, i, head_dim, rotated, position, theta) : x[e];
      uint16_t *row = row_of(L, st == 0 ? c0 : c1, st == 0 ? p0 : p1, position, h);
      row[i] = narrow_cache(v, cache_bf16);
    }
  }
  return 0;
}

int fkref_step_store(const float *x0, const float *x1, uint16_t *c0, uint16_t *c1, int n_stores, int rope0,
                     int rope1, int kv_heads, int head_dim, int length, int slots, int rotated, float theta,
                     uint32_t position, uint32_t slot, int cache_bf16) {
  if (slot >= (uint32_t)slots) return 0;
  fkref_rows L = {0, kv_heads, head_dim, length, slot, 0, 0, 0, NULL};
  return store_rows(&L, x0, x1, c0, c1, NULL, NULL, n_stores, rope0, rope1, rotated, theta, position, cache_bf16);
}

/* The store into a paged pool: `table` the row's block table of `table_len`
 * blocks; nothing stored for a position past the table or a block past the
 * pool. */
int fkref_step_store_paged(const float *x0, const float *x1, uint16_t *const *p0, uint16_t *const *p1,
                           int n_stores, int rope0, int rope1, int kv_heads, int head_dim, int block_size,
                           const uint32_t *table, int table_len, int blocks, int rotated, float theta,
                           uint32_t position, int cache_bf16) {
  if (block_size <= 0 || table_len <= 0 || blocks <= 0) return -1;
  if (position / (uint32_t)block_size >= (uint32_t)table_len ||
      table[position / (uint32_t)block_size] >= (uint32_t)blocks)
    return 0;
  fkref_rows L = {1, kv_heads, head_dim, 0, 0, block_size, table_len, blocks, table};
  return store_rows(&L, x0, x1, NULL, NULL, p0, p1, n_stores, rope0, rope1, rotated, theta, position, cache_bf16);
}

#define SPLIT_MAX 128
#define ATTEND_CHUNKS 8

/* The pairwise sum of n values (n a power of two): the halves' sums added,
 * ((a0 + a1) + (a2 + a3)) + ... */
static float pairwise_sum(const float *a, int n) {
  if (n == 1) return a[0];
  return pairwise_sum(a, n / 2) + pairwise_sum(a + n / 2, n / 2);
}

static int attend_rows(const fkref_rows *L, const float *q, const uint16_t *kc, const uint16_t *vc,
                       uint16_t *const *kp, uint16_t *const *vp, float *partials, int heads, int kv_heads,
                       int head_dim, int splits, int split, int rope, int rotated, float theta, float scale,
                       int window, uint32_t position, uint32_t reach, int cache_bf16) {
  const int group = heads / kv_heads;
  const int d = head_dim;
  const uint32_t SPLIT = (uint32_t)split;
  if (group > 8 || d > 64 || d % 8 || split < ATTEND_CHUNKS || split > SPLIT_MAX || split % ATTEND_CHUNKS) return -1;
  if ((split / ATTEND_CHUNKS) & (split / ATTEND_CHUNKS - 1)) return -1; /* runs of a power of two */
  float qs[8 * 64];
  float wt[8 * SPLIT_MAX];
  float mx[8];
  uint32_t first = (window && position + 1 > (uint32_t)window) ? position + 1 - (uint32_t)window : 0;
  /* The last position read: the row's own, or its reach past it. */
  const uint32_t top = reach > position ? reach : position;
  for (int g = 0; g < kv_heads; g++) {
    for (int t = 0; t < splits; t++) {
      uint32_t lo = (uint32_t)t * SPLIT > first ? (uint32_t)t * SPLIT : first;
      uint32_t hi = top + 1 < (uint32_t)(t + 1) * SPLIT ? top + 1 : (uint32_t)(t + 1) * SPLIT;
      int count = hi > lo ? (int)(hi - lo) : 0;
      for (int e = 0; e < group * d; e++) {
        const float *head = q + (size_t)(g * group + e / d) * d;
        qs[e] = rope ? fkref_rope_elem(head, e % d, d, rotated, position, theta) : head[e % d];
      }
      /* A score: four fused multiply-add chains from +0, one a quarter of
       * the dimensions in order, added ((c0 + c1) + (c2 + c3)), then scaled. */
      const int dq = d / 4;
      for (int h = 0; h < group; h++) {
        for (int r = 0; r < count; r++) {
          const uint16_t *kr = row_of(L, (uint16_t *)kc, kp, lo + (uint32_t)r, g);
          float c[4];
          for (int j = 0; j < 4; j++) {
            c[j] = 0.0f;
            for (int i = j * dq; i < (j + 1) * dq; i++)
              c[j] = fmaf(qs[h * d + i], widen_cache(kr[i], cache_bf16), c[j]);
          }
          wt[h * SPLIT + r] = ((c[0] + c[1]) + (c[2] + c[3])) * scale;
        }
      }
      for (int h = 0; h < group; h++) {
        float m = -INFINITY;
        for (int r = 0; r < count; r++) m = fkref_max(m, wt[h * SPLIT + r]);
        mx[h] = m;
      }
      for (int h = 0; h < group; h++)
        for (int r = 0; r < count; r++) wt[h * SPLIT + r] = fkref_exp(wt[h * SPLIT + r] - mx[h]);
      /* The weights' sum and the weighted values over the split's positions
       * in ATTEND_CHUNKS runs of split / ATTEND_CHUNKS: a run's weights by
       * pairwise_sum (a position past `count` adding +0), its values in order
       * of position from +0 (acc = fma(w, v, acc)); then the runs' sums
       * added in order from +0. */
      const int run = split / ATTEND_CHUNKS;
      float runw[SPLIT_MAX / ATTEND_CHUNKS];
      for (int h = 0; h < group; h++) {
        /* Partials: acc[heads][splits][d], then [heads][splits][max, sum]. */
        const size_t ht = (size_t)(g * group + h) * splits + t;
        float *out = partials + ht * d;
        float *stat = partials + (size_t)heads * splits * d + 2 * ht;
        for (int i = 0; i < d; i++) {
          float l = 0.0f;
          float acc = 0.0f;
          for (int c = 0; c < ATTEND_CHUNKS; c++) {
            for (int u = 0; u < run; u++) runw[u] = c * run + u < count ? wt[h * SPLIT + c * run + u] : 0.0f;
            float lc = pairwise_sum(runw, run);
            float ac = 0.0f;
            for (int r = c * run; r < (c + 1) * run && r < count; r++) {
              const uint16_t *vr = row_of(L, (uint16_t *)vc, vp, lo + (uint32_t)r, g);
              ac = fmaf(wt[h * SPLIT + r], widen_cache(vr[i], cache_bf16), ac);
            }
            l = l + lc;
            acc = acc + ac;
          }
          if (i == 0) {
            stat[0] = mx[h];
            stat[1] = l;
          }
          out[i] = acc;
        }
      }
    }
  }
  return 0;
}

int fkref_step_attend(const float *q, const uint16_t *kc, const uint16_t *vc, float *partials, int heads,
                      int kv_heads, int head_dim, int length, int slots, int splits, int split, int rope,
                      int rotated, float theta, float scale, int window, uint32_t position, uint32_t slot,
                      int cache_bf16) {
  fkref_rows L = {0, kv_heads, head_dim, length, slot < (uint32_t)slots ? slot : 0, 0, 0, 0, NULL};
  return attend_rows(&L, q, kc, vc, NULL, NULL, partials, heads, kv_heads, head_dim, splits, split, rope, rotated,
                     theta, scale, window, position, position, cache_bf16);
}

/* The ring attention with a reach: positions up to max(position, reach). */
int fkref_step_attend_reach(const float *q, const uint16_t *kc, const uint16_t *vc, float *partials, int heads,
                            int kv_heads, int head_dim, int length, int slots, int splits, int split, int rope,
                            int rotated, float theta, float scale, int window, uint32_t position, uint32_t slot,
                            uint32_t reach, int cache_bf16) {
  fkref_rows L = {0, kv_heads, head_dim, length, slot < (uint32_t)slots ? slot : 0, 0, 0, 0, NULL};
  return attend_rows(&L, q, kc, vc, NULL, NULL, partials, heads, kv_heads, head_dim, splits, split, rope, rotated,
                     theta, scale, window, position, reach, cache_bf16);
}

/* The attention over a paged pool: the row's block table `table` of
 * `table_len` blocks, the pool's `blocks` blocks at kp[b] and vp[b]. */
int fkref_step_attend_paged(const float *q, uint16_t *const *kp, uint16_t *const *vp, float *partials, int heads,
                            int kv_heads, int head_dim, int block_size, const uint32_t *table, int table_len,
                            int blocks, int splits, int split, int rope, int rotated, float theta, float scale,
                            int window, uint32_t position, uint32_t reach, int cache_bf16) {
  if (block_size <= 0 || table_len <= 0 || blocks <= 0) return -1;
  fkref_rows L = {1, kv_heads, head_dim, 0, 0, block_size, table_len, blocks, table};
  return attend_rows(&L, q, NULL, NULL, kp, vp, partials, heads, kv_heads, head_dim, splits, split, rope, rotated,
                     theta, scale, window, position, reach, cache_bf16);
}

/* The attention in wide splits (fk_attention.h, attend_wide): a split of S =
 * 64 W positions taken by W runs of 64 (W <= 8); in each run, for each query
 * head, the score of position r is its fma chain from +0 over the dimensions
 * in order, times scale (-inf off the split); the run's maximum m; weights
 * exp(score - m) binary64's rounded once; their sum by the pairwise tree over
 * the run's positions in order (pairs r, r ^ 1, then pairs of pairs, ...);
 * for each dimension the fma chain over r of weight * value; then the runs
 * merged in order by exp(m_run - M).  Reads the caches as they stand (the
 * store, if any, is the caller's). */
int fkref_step_attend_wide(const float *q, const uint16_t *kc, const uint16_t *vc, float *partials, int heads,
                           int kv_heads, int head_dim, int length, int slots, int splits, int split, int rope,
                           int rotated, float theta, float scale, int window, uint32_t position, uint32_t slot,
                           int cache_bf16) {
  const int group = kv_heads > 0 ? heads / kv_heads : 0;
  const int d = head_dim;
  const int W = split / 64;
  if (group < 1 || group > 8 || heads % kv_heads || (d != 16 && d != 32 && d != 64) || split % 64 || W < 1 ||
      W > 8)
    return -1;
  uint32_t s = slot < (uint32_t)slots ? slot : 0;
  uint32_t first = (window && position + 1 > (uint32_t)window) ? position + 1 - (uint32_t)window : 0;
  float qs[8 * 64], kf[64][64], vf[64][64], sc[64], e[64], bt[64];
  float mw[8][8], lw[8][8], aw[8][8][64];
  for (int g = 0; g < kv_heads; g++) {
    for (int h = 0; h < group; h++)
      for (int j = 0; j < d; j++) {
        const float *head = q + (size_t)(g * group + h) * d;
        qs[h * d + j] = rope ? fkref_rope_elem(head, j, d, rotated, position, theta) : head[j];
      }
    for (int t = 0; t < splits; t++) {
      uint32_t lo = (uint32_t)t * split > first ? (uint32_t)t * split : first;
      uint32_t hi = position + 1 < (uint32_t)(t + 1) * split ? position + 1 : (uint32_t)(t + 1) * split;
      const size_t base = ((size_t)s * kv_heads + g) * length;
      for (int w = 0; w < W; w++) {
        uint32_t run0 = (uint32_t)t * split + 64u * w;
        int live[64];
        for (int r = 0; r < 64; r++) {
          uint32_t at = run0 + r;
          live[r] = at >= lo && at < hi;
          uint32_t ring = (live[r] ? at : (hi > lo ? lo : 0)) % (uint32_t)length;
          for (int i = 0; i < d; i++) {
            kf[r][i] = widen_cache(kc[(base + ring) * d + i], cache_bf16);
            vf[r][i] = live[r] ? widen_cache(vc[(base + ring) * d + i], cache_bf16) : 0.0f;
          }
        }
        for (int h = 0; h < group; h++) {
          float m = -INFINITY;
          for (int r = 0; r < 64; r++) {
            float c = 0.0f;
            for (int i = 0; i < d; i++) c = fmaf(qs[h * d + i], kf[r][i], c);
            sc[r] = live[r] ? c * scale : -INFINITY;
            m = fkref_max(m, sc[r]);
          }
          for (int r = 0; r < 64; r++) e[r] = m == -INFINITY ? 0.0f : fkref_exp(sc[r] - m);
          for (int r = 0; r < 64; r++) bt[r] = e[r];
          for (int width = 1; width < 64; width <<= 1)
            for (int r = 0; r < 64; r += 2 * width) bt[r] = bt[r] + bt[r + width];
          mw[w][h] = m;
          lw[w][h] = bt[0];
          for (int i = 0; i < d; i++) {
            float acc = 0.0f;
            for (int r = 0; r < 64; r++) acc = fmaf(e[r], vf[r][i], acc);
            aw[w][h][i] = acc;
          }
        }
      }
      for (int h = 0; h < group; h++) {
        float M = -INFINITY;
        for (int w = 0; w < W; w++) M = fkref_max(M, mw[w][h]);
        const size_t ht = (size_t)(g * group + h) * splits + t;
        for (int i = 0; i < d; i++) {
          float L = 0.0f, A = 0.0f;
          if (M != -INFINITY) {
            for (int w = 0; w < W; w++) {
              float ew = mw[w][h] == -INFINITY ? 0.0f : fkref_exp(mw[w][h] - M);
              float lp = lw[w][h] * ew;
              float ap = aw[w][h][i] * ew;
              L = L + lp;
              A = A + ap;
            }
          }
          partials[ht * d + i] = A;
          if (i == 0) {
            float *st = partials + (size_t)heads * splits * d + 2 * ht;
            st[0] = M;
            st[1] = L;
          }
        }
      }
    }
  }
  return 0;
}

int fkref_step_combine(const float *partials, float *out, int heads, int head_dim, int splits) {
  for (int h = 0; h < heads; h++) {
    const float *ph = partials + (size_t)h * splits * head_dim;
    const float *st = partials + (size_t)heads * splits * head_dim + (size_t)h * splits * 2;
    float m = -INFINITY;
    for (int t = 0; t < splits; t++) m = fkref_max(m, st[2 * t]);
    for (int i = 0; i < head_dim; i++) {
      float l = 0.0f;
      float acc = 0.0f;
      for (int t = 0; t < splits; t++) {
        float w = fkref_exp(st[2 * t] - m);
        l = l + st[2 * t + 1] * w;
        acc = acc + ph[(size_t)t * head_dim + i] * w;
      }
      out[(size_t)h * head_dim + i] = acc / l;
    }
  }
  return 0;
}

uint32_t fkref_argmax(const float *x, int n) {
  uint32_t best = 0;
  for (int i = 1; i < n; i++)
    if (x[i] > x[best]) best = (uint32_t)i;
  return best;
}

uint64_t fkref_argmax_key(float v, uint32_t index) {
  uint32_t hi;
  if (isnan(v)) {
    hi = index == 0 ? 0xFFFFFFFFu : 0u;
  } else {
    uint32_t b = 0;
    if (v != 0.0f) memcpy(&b, &v, 4);
    hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - index);
}

/* Routing (fk_step_route): the k largest logits by their argmax keys (a
 * NaN's key the lowest, its index's), then exp(x_r - x_0) binary64's rounded
 * once, their sum from +0 in rank order, each over the sum, times its
 * expert's scale if given. */
int fkref_route(const float *x, const float *scale, uint32_t *ids, float *ws, int n, int k, int has_scale) {
  if (k < 1 || k > 8 || k > n) return -1;
  uint32_t taken[8];
  float tv[8], e[8], total = 0.0f;
  for (int r = 0; r < k; r++) {
    uint64_t best = 0;
    for (int i = 0; i < n; i++) {
      int seen = 0;
      for (int q = 0; q < r; q++) seen |= taken[q] == (uint32_t)i;
      uint64_t key = isnan(x[i]) ? (uint64_t)(0xFFFFFFFFu - (uint32_t)i) : fkref_argmax_key(x[i], (uint32_t)i);
      if (!seen && key > best) best = key;
    }
    taken[r] = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu);
    tv[r] = x[taken[r]];
  }
  for (int r = 0; r < k; r++) {
    e[r] = fkref_exp(tv[r] - tv[0]);
    total = total + e[r];
  }
  for (int r = 0; r < k; r++) {
    float w = e[r] / total;
    if (has_scale) w = w * scale[taken[r]];
    ids[r] = taken[r];
    ws[r] = w;
  }
  return 0;
}

/* CombineRanks (fk_step_combine_ranks): a left fold from the first rank's
 * product, each product rounded, then the residual added in front. */
int fkref_combine_ranks(const float *w, const float *x, const float *res, float *y, int seg, int ranks,
                        int residual) {
  if (ranks < 1 || seg < 1) return -1;
  for (int i = 0; i < seg; i++) {
    float acc = w[0] * x[i];
    for (int r = 1; r < ranks; r++) {
      float t = w[r] * x[(size_t)r * seg + i];
      acc = acc + t;
    }
    y[i] = residual ? res[i] + acc : acc;
  }
  return 0;
}

uint64_t fkref_argmax_keyed(const float *x, int n) {
  uint64_t best = 0;
  for (int i = 0; i < n; i++) {
    uint64_t k = fkref_argmax_key(x[i], (uint32_t)i);
    if (k > best) best = k;
  }
  return best;
}

/* ------------------------------------------------------------------------ */
/* Element-wise numerics for the IR interpreter                              */

void fkref_widen_f16_n(const uint16_t *h, float *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = fkref_widen_f16(h[i]);
}

void fkref_widen_bf16_n(const uint16_t *b, float *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = fkref_widen_bf16(b[i]);
}

void fkref_narrow_f16_n(const float *x, uint16_t *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = fkref_narrow_f16(x[i]);
}

void fkref_narrow_bf16_n(const float *x, uint16_t *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = fkref_narrow_bf16(x[i]);
}

void fkref_narrow_f16_f64_n(const double *x, uint16_t *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = fkref_narrow_f16_f64(x[i]);
}

/* IEEE 754's fusedMultiplyAdd: C's fmaf rounds the exact a * b + c once
 * (Interp.hs:872-891); a NaN result is the quiet NaN with no payload. */
void fkref_fma_f32_n(const float *a, const float *b, const float *c, float *y, size_t n) {
  for (size_t i = 0; i < n; i++) {
    const float r = fmaf(a[i], b[i], c[i]);
    y[i] = isnan(r) ? float_of(0x7FC00000u) : r;
  }
}

void fkref_unary_f64_n(int op, const double *x, double *y, size_t n) {
  for (size_t i = 0; i < n; i++) {
    switch (op) {
      case FKREF_RSQRT: y[i] = 1.0 / sqrt(x[i]); break;
      case FKREF_EXP: y[i] = exp(x[i]); break;
      case FKREF_LOG: y[i] = log(x[i]); break;
      default: y[i] = tanh(x[i]); break;
    }
  }
}
