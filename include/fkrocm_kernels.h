/*
 * fkrocm_kernels.h — the parameter structs of the target's gfx950 kernels,
 * in C layout: what a launch's kernarg carries after its buffers' addresses
 * (src/FuryKernel/Abi.hs:113-133, a kernel's one parameter struct laid out
 * as C lays out a struct of its fields).  The kernels include this header,
 * so the device code and every binding read one definition; the manifest
 * (fkrocm.h, `fk_manifest_*`) describes each kernel's buffers and these
 * fields with their offsets, and its ABI hash covers both.
 *
 * Entry names and their buffers in binding order:
 *   fk_step_gemv_<f16|f32>_k<K>_r<R>_p<PRO>_e<EPI>
 *       w0 w1 w2 y0 y1 y2 src src2 gamma table token res res_table res_token
 *       epi_out arg                                    fk_step_gemv_params
 *   fk_step_token        arg out token position       fk_step_token_params
 *   fk_step_store        x0 x1 c0 c1 position slot rope
 *                                                      fk_step_store_params
 *   fk_step_attend       q knew vnew kc vc position slot rope partials reach
 *                                                      fk_step_attend_params
 *   fk_step_attend_paged q knew vnew kpool vpool position table rope partials reach
 *                                                      fk_step_attend_paged_params
 *   fk_step_store_paged  x0 x1 p0 p1 position table rope
 *                                                      fk_step_store_paged_params
 *   fk_step_combine      partials out                 fk_step_combine_params
 *   fk_gemm_f16_<store|add|silu_mul>  a b0 b1 b2 c0 c1 c2 r0   fk_gemm_params
 *   fk_gemm_f16_qkv_rope a b0 b1 b2 c0 c1 c2 r0 position slot rope
 *                                                      fk_gemm_qkv_params
 *   fk_gemm_f16_store_keys a b0 b1 b2 c0 c1 c2 r0 keys  fk_gemm_params
 *   fk_gemm_f16_qkv_rope_paged a b0 b1 b2 c0 c1 c2 r0 position table rope
 *                                                      fk_gemm_qkv_paged_params
 *   fk_prefill_attend_g<1|2|4>, fk_prefill_attend_f16_g<1|2|4>
 *                        qr kc vc position slot out ks vs
 *                                                      fk_prefill_attend_params
 *     (the f16 form: f16 rings and no staged rows, each key block loaded
 *     straight into LDS; ks and vs unused)
 *   fk_prefill_attend_paged_g<1|2|4>, fk_prefill_attend_paged_f16_g<1|2|4>
 *                        qr kc vc position table out   fk_prefill_attend_paged_params
 *     (the f16 form: f16 pools under 4 GiB, tables of at most 256 blocks,
 *     each key block loaded straight into LDS)
 *   fk_prefill_argmax_keys keys out                    fk_prefill_argmax_keys_params
 *   (the manifest lists every entry.)
 */
#ifndef FKROCM_KERNELS_H
#define FKROCM_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The GEMV step (a planned step of one row: Plan.hs:17-31). ---------------- */

/* Prologue modes: how a GEMV step's threadgroups make the anchors' input row.
 * An entry's `_p<mode>` suffix is the mode it runs; its parameter struct's
 * pro_mode must agree (the launch table refuses it otherwise). */
enum {
  FK_PRO_STORED = 0,         /* x = src */
  FK_PRO_RMSNORM = 1,        /* x = rmsnorm(src) * gamma * factor */
  FK_PRO_GATHER = 2,         /* x = table[token] * gfactor */
  FK_PRO_GATHER_RMSNORM = 3, /* x = rmsnorm(table[token] * gfactor) * gamma * factor */
  FK_PRO_SILU_MUL = 4,       /* x = act(src) * src2[src2_off ..] (act: FK_ACT_*, SiLU or GELU-tanh) */
  FK_PRO_COMBINE = 5         /* x = the attention's combine of the partials at src (at most 8 splits): the
                                plan's Combine step folded into the GEMV step that reads its output */
};

/* Epilogue modes, on the anchors' tile (the entry's `_e<mode>` suffix). */
enum {
  FK_EPI_NONE = 0,
  FK_EPI_ADD_STORED = 1, /* out = res + tile */
  FK_EPI_ADD_GATHER = 2, /* out = table[token] * gfactor + tile */
  FK_EPI_SILU_MUL = 3,   /* out = act(tile of anchor 0) * tile of anchor 1 (act: FK_ACT_*) */
  FK_EPI_ARGMAX = 4,     /* arg = max(arg, argmax key of each row) (the greedy token, folded in) */
  FK_EPI_SOFTCAP = 5     /* out = cap tanh(tile / cap); with arg_slots, also the argmax keys of out */
};

/* The activation of an act·mul (src/FuryKernel/Program/Graph.hs:287-291): the
 * GEMV step's act·mul prologue and epilogue, the light act·mul step, the
 * prefill GEMM's act·mul epilogue. */
enum {
  FK_ACT_SILU = 0,     /* a / (1 + e^-a) */
  FK_ACT_GELU_TANH = 1 /* 0.5 a (1 + tanh(sqrt(2/pi) (a + 0.044715 a^3))) */
};

typedef struct fk_step_gemv_params {
  uint32_t n_anchors;    /* 1 to 3 */
  uint32_t rows[3];      /* each anchor's outputs */
  uint32_t first_row[4]; /* anchor j's rows are [first_row[j], first_row[j + 1]) of the numbered rows */
  uint32_t k;            /* the input row's width */
  uint32_t pro_mode;
  uint32_t seg;          /* RMSNorm's segment: the row (k) */
  float eps;
  float factor;          /* RMSNorm's factor */
  float gfactor;         /* the gather's factor */
  uint32_t has_gamma;
  uint32_t epi_mode;
  uint32_t store_tile;   /* the anchors' own values are stored (into y[j]) */
  uint32_t table_rows;   /* the gathered table's rows: a token past them reads its last */
  uint32_t blocks;       /* row blocks */
  uint32_t arg_slots;    /* the argmax epilogue's slots (one a threadgroup); a threadgroup past them stores none */
  uint32_t act;          /* the act·mul prologue's and epilogue's activation (FK_ACT_*) */
  uint32_t src2_off;     /* elements into src2 where the act·mul prologue's second row starts */
  float cap;             /* the softcap epilogue's cap (positive, finite) */
  uint32_t splits;       /* the combine prologue's partials: splits a head (at most 8) */
  uint32_t head_dim;     /* ... and the heads' width (k / head_dim heads, a multiple of 4) */
} fk_step_gemv_params;

typedef struct fk_step_token_params {
  uint32_t slots;   /* the folded argmax's slots: one a threadgroup of the logits' step */
  uint32_t context; /* positions wrap below this */
  uint32_t step;    /* positions advance by this (0 holds the position) */
  uint32_t advance; /* also set the next step's token and position */
} fk_step_token_params;

/* KV stores, decode attention and its combine (Eval.hs:415-527). ---------- */

typedef struct fk_step_store_params {
  uint32_t n_stores;   /* 1 or 2 */
  uint32_t rope[2];    /* store j's value is RoPE'd first */
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t length;     /* the ring's positions */
  uint32_t slots;      /* the ring's sequences */
  uint32_t rotated;    /* pairs turned */
  uint32_t rope_rows;  /* positions the RoPE table holds */
  uint32_t cache_bf16; /* the caches round to bf16 (else f16) */
} fk_step_store_params;

typedef struct fk_step_attend_params {
  uint32_t heads;
  uint32_t kv_heads;
  uint32_t head_dim; /* a multiple of 8, at most 64 */
  uint32_t length;   /* the ring's positions */
  uint32_t slots;
  uint32_t splits;   /* threadgroups per kv head */
  uint32_t split;    /* positions a split covers: split t is [t split, (t + 1) split); 64 or 128 */
  uint32_t rope;     /* q is RoPE'd first */
  uint32_t rotated;
  uint32_t rope_rows;
  float scale;       /* the attention's scale, rounded once to binary32 */
  uint32_t window;   /* 0: none */
  uint32_t cache_bf16;
  uint32_t store;    /* the new key and value rows are stored into the caches first */
  uint32_t krope;    /* the stored key row is RoPE'd first (q's table) */
  uint32_t has_reach; /* positions up to max(position, reach[0]) (Graph.hs:223-247); else up to position */
} fk_step_attend_params;

/* A paged pool (Graph.hs:144-152): blocks of block_size positions, each an
 * array of its own at the address pool[b] (an array of the blocks' device
 * addresses); position t, kv head h of a row at (h block_size + t mod
 * block_size) head_dim in block table[t / block_size] of the row's block
 * table.  A table index past table_len or a block past `blocks` is clamped
 * into them (the gate keeps a valid program's inside). */
typedef struct fk_paging {
  uint32_t block_size;
  uint32_t table_len;  /* blocks a row's table lists */
  uint32_t blocks;     /* the pool's blocks */
} fk_paging;

/* fk_step_attend_paged: the attention over paged pools (`a.length` the
 * positions the table covers, table_len block_size; `a.slots` unused). */
typedef struct fk_step_attend_paged_params {
  fk_step_attend_params a;
  fk_paging g;
} fk_step_attend_paged_params;

/* fk_step_store_paged: the KV store into paged pools (`s.length` and
 * `s.slots` unused). */
typedef struct fk_step_store_paged_params {
  fk_step_store_params s;
  fk_paging g;
} fk_step_store_paged_params;

typedef struct fk_step_combine_params {
  uint32_t heads;
  uint32_t head_dim;
  uint32_t splits;
} fk_step_combine_params;

typedef struct fk_step_argmax_params {
  uint32_t n;
} fk_step_argmax_params;

typedef struct fk_step_act_mul_params {
  uint32_t n;
  uint32_t act;   /* FK_ACT_* */
  uint32_t b_off; /* elements into b where the second row starts (a gated activation's second half) */
  uint32_t half;  /* 0: a and b as rows; else segments of 2 half of one row a (b unread): y[s half + i] =
                     act(a[2 s half + i]) a[2 s half + half + i] (GatedGelu, Eval.hs:356-371) */
} fk_step_act_mul_params;

/* Routing (Eval.hs:391-404, routeRow :648-655): the k largest of n logits,
 * ties to the lower index (a NaN ranked below every number), in rank order;
 * their weights exp(x - best) binary64's rounded once over their sum from
 * +0 in rank order, each divided by the sum, times its expert's scale if
 * has_scale. */
typedef struct fk_step_route_params {
  uint32_t n;
  uint32_t k; /* 1 to 8, at most n */
  uint32_t has_scale;
} fk_step_route_params;

/* LinearRouted (Eval.hs:291-321): for each of `ranks` ranks, the n rows of
 * the table entry ids[rank] (its address table[ids[rank]], the id clamped
 * below `entries`) times the row x (shared) or the rank's slice of k
 * elements, in the reference GEMV's order; a rank's rows in
 * groups_per_rank threadgroups. */
typedef struct fk_gemv_routed_params {
  uint32_t n;
  uint32_t k;
  uint32_t ranks;
  uint32_t shared;
  uint32_t entries;
  uint32_t groups_per_rank;
} fk_gemv_routed_params;

/* CombineRanks (Eval.hs:405-414): y[i] = ((w0 x0[i] + w1 x1[i]) + ...), x_r
 * the rank's segment of `seg`; then, with `residual`, res[i] + y[i] (the
 * residual add the plan recomputes with it). */
typedef struct fk_step_combine_ranks_params {
  uint32_t seg;
  uint32_t ranks;
  uint32_t residual;
} fk_step_combine_ranks_params;

/* A light step's elementwise value of stored rows, one thread an element of
 * the n = rows * width elements (Eval.hs:336-355, 536-544):
 *   FK_ELT_ADD          y = a + b                      (Add)
 *   FK_ELT_SCALE        y = a * b[0]                   (ScaleBy; b the weight widened to f32)
 *   FK_ELT_STANDARDIZE  y[j] = (factor a[j] - b[j]) c[j], j the element's place in its row
 *                       (Standardize; b the bias, c the scale, each of `width` f32)
 *   FK_ELT_CONCAT       rows of width of a, then width_b of b (Concat; n the output's elements) */
enum { FK_ELT_ADD = 0, FK_ELT_SCALE = 1, FK_ELT_STANDARDIZE = 2, FK_ELT_CONCAT = 3 };
typedef struct fk_step_elementwise_params {
  uint32_t n;
  uint32_t op;      /* FK_ELT_* */
  uint32_t width;   /* a row's elements (of a, for FK_ELT_CONCAT) */
  uint32_t width_b; /* FK_ELT_CONCAT: a row's elements of b */
  float factor;     /* FK_ELT_STANDARDIZE */
} fk_step_elementwise_params;

/* Gather (Eval.hs:528-535): row r of y is the sum, from +0 in order, of the
 * table rows of its `count` tokens (each clamped below table_rows), times
 * factor: y[r][j] = (Σ_t table[tok(r, t)][j]) f.  One thread an element. */
typedef struct fk_step_gather_params {
  uint32_t rows;
  uint32_t width;
  uint32_t count;      /* tokens a row */
  uint32_t table_rows;
  float factor;
} fk_step_gather_params;

typedef struct fk_step_advance_params {
  uint32_t context; /* positions wrap below this */
  uint32_t step;    /* positions advance by this (0 holds the position) */
} fk_step_advance_params;

typedef struct fk_init_normal_params {
  uint64_t count;
  uint64_t seed;
  float std;
  uint32_t dtype; /* what is stored: 0 binary32, 1 binary16, 2 bfloat16 (each the value rounded once) */
} fk_init_normal_params;

/* Standalone kernels. ----------------------------------------------------- */

typedef struct fk_gemv_params {
  uint32_t n; /* rows of W (outputs) */
  uint32_t k; /* columns of W (inputs), a multiple of the pack */
} fk_gemv_params;

typedef struct fk_rmsnorm_params {
  uint32_t rows;  /* rows of x */
  uint32_t width; /* elements per row */
  uint32_t seg;   /* elements per segment (a multiple of 4 dividing width) */
  float eps;      /* rounded once to binary32 */
  float factor;   /* a constant factor; 1 multiplies by nothing */
  uint32_t has_gamma;
} fk_rmsnorm_params;

typedef struct fk_softmax_params {
  uint32_t rows;
  uint32_t n; /* elements per row, a multiple of 4 */
} fk_softmax_params;

typedef struct fk_fill_params {
  uint32_t count; /* 32-bit words */
  uint32_t value;
} fk_fill_params;

typedef struct fk_noop_params {
  uint32_t unused;
} fk_noop_params;

typedef struct fk_stream_read_params {
  uint64_t words; /* 16-byte words to read */
} fk_stream_read_params;

/* The prefill (steps of many rows, Tile.hs:76-157). ----------------------- */

enum {
  FK_GEMM_STORE = 0,    /* C = A B^T (f32 rows) */
  FK_GEMM_ADD = 1,      /* C = R + A B^T (f32 rows), R [M, ldc]; R may be C */
  FK_GEMM_SILU_MUL = 2, /* C = f16(silu(A G^T) (A U^T)) in the tile layout; B0 the paired gate/up weights */
  FK_GEMM_QKV_ROPE = 3, /* anchors q, k, v: q RoPE'd into f16 rows (C0), k RoPE'd into the K cache (C1), v into
                           the V cache (C2), at each row's slot and position */
  FK_GEMM_STORE_KEYS = 4, /* one anchor's C = A B^T (f32 rows), and for each row and 128 columns the greedy
                             token's 64-bit key of their largest element: keys [M][N / 128] */
  FK_GEMM_QKV_ROPE_PAGED = 5 /* FK_GEMM_QKV_ROPE with the caches paged pools, through each row's block table */
};

typedef struct fk_gemm_params {
  uint32_t m;            /* rows of A and C, a multiple of 256 */
  uint32_t k;            /* a multiple of 64 */
  uint32_t n_anchors;    /* 1 to 3 weights (SiLU·mul: 1, the pair) */
  uint32_t first_col[4]; /* anchor j's columns of C are [first_col[j], first_col[j + 1]), each a multiple of 256 */
  uint32_t ldc[3];       /* row stride of anchor j's output (its columns; SiLU·mul: N, gate's rows) */
  uint32_t act;          /* the act·mul epilogue's activation (FK_ACT_*) */
} fk_gemm_params;

typedef struct fk_gemm_rope_params {
  uint32_t kv_heads;
  uint32_t rope_rows; /* positions the RoPE table holds */
  uint32_t length;    /* ring length */
  uint32_t slots;
  uint32_t cache_bf16;
  uint32_t staged;    /* k and v rows into staging rows [rows][kv_heads][64] (the plan's staged stores) */
} fk_gemm_rope_params;

typedef struct fk_gemm_qkv_params {
  fk_gemm_params g;
  fk_gemm_rope_params r;
} fk_gemm_qkv_params;

/* fk_gemm_f16_qkv_rope_paged: `r.length` and `r.slots` unused, no staged rows. */
typedef struct fk_gemm_qkv_paged_params {
  fk_gemm_params g;
  fk_gemm_rope_params r;
  fk_paging pg;
} fk_gemm_qkv_paged_params;

typedef struct fk_prefill_gather_params {
  uint32_t rows;
  uint32_t width;      /* a multiple of 4 */
  uint32_t table_rows;
  uint32_t table_f16;  /* the table is f16 (else f32) */
  float factor;
} fk_prefill_gather_params;

typedef struct fk_prefill_norm_params {
  uint32_t rows;  /* a multiple of 256 */
  uint32_t width; /* a multiple of 32 */
  float eps;
  float factor;
  uint32_t has_gamma;
} fk_prefill_norm_params;

typedef struct fk_prefill_rope_params {
  uint32_t rows;
  uint32_t heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t rotated;   /* pairs RoPE turns */
  uint32_t rope_rows; /* positions the RoPE table holds */
  uint32_t length;    /* ring length */
  uint32_t slots;
  uint32_t cache_bf16;
  uint32_t staged;    /* kc and vc are staging rows [rows][kv_heads][head_dim], the row's own */
} fk_prefill_rope_params;

/* fk_prefill_rope_store_paged: `r.length`, `r.slots` and `r.staged` unused. */
typedef struct fk_prefill_rope_paged_params {
  fk_prefill_rope_params r;
  fk_paging g;
} fk_prefill_rope_paged_params;

typedef struct fk_prefill_attend_params {
  uint32_t rows;     /* a multiple of 32 */
  uint32_t heads;
  uint32_t kv_heads; /* heads / kv_heads (G) is 1, 2 or 4 */
  uint32_t length;   /* ring length, a multiple of 64 */
  uint32_t slots;
  uint32_t window;   /* 0: none; else a row sees positions > position - window */
  uint32_t cache_bf16;
  float scale;
  uint32_t staged;   /* a sequence's positions from its run's first row on are read from ks and vs */
  uint32_t run_rows; /* each sequence's run of rows in the step, a multiple of 32 dividing rows (0: one run);
                       staged runs read their own rows from ks and vs */
} fk_prefill_attend_params;

/* fk_prefill_attend_paged_g*: the attention over paged pools; `a.slots`,
 * `a.staged` and `a.run_rows` unused, `a.length` the positions a table covers
 * (table_len block_size). */
typedef struct fk_prefill_attend_paged_params {
  fk_prefill_attend_params a;
  fk_paging g;
} fk_prefill_attend_paged_params;

/* The staged rows landed in the ring (src/FuryKernel/Program/Plan.hs:41-50):
 * row r's kv heads from ks and vs ([rows][kv_heads][head_dim]) into kc and
 * vc at (slot[r], head, position[r] mod length). */
typedef struct fk_prefill_land_params {
  uint32_t rows;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t length;
  uint32_t slots;
} fk_prefill_land_params;

typedef struct fk_prefill_softcap_params {
  uint32_t count; /* elements */
  float cap;
} fk_prefill_softcap_params;

typedef struct fk_prefill_argmax_params {
  uint32_t rows;
  uint32_t width;
} fk_prefill_argmax_params;

typedef struct fk_prefill_argmax_keys_params {
  uint32_t rows;
  uint32_t parts; /* keys a row (fk_gemm_f16_store_keys: its columns / 128) */
} fk_prefill_argmax_keys_params;

#ifdef __cplusplus
}
#endif

#endif /* FKROCM_KERNELS_H */
