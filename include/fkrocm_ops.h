/*
 * fkrocm_ops.h — whole operations as one C call each, over device buffers
 * the caller holds: for callers that want an operation rather than a launch
 * table of their own.
 *
 * The decode attention step over a ring KV cache: the new key and value rows
 * stored at the row's position (the key RoPE'd), the attention of each query
 * head over its kv head's positions in splits, and the combine of the splits
 * — the planned step's KvStore effects, Partials anchor and Combine
 * (src/FuryKernel/Program/Eval.hs:415-527, src/FuryKernel/Program/Plan.hs:
 * 174-181), with the same kernels and bits as the planned step's launches.
 */
#ifndef FKROCM_OPS_H
#define FKROCM_OPS_H

#include "fkrocm.h"
#include "fkrocm_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Device addresses (16-byte aligned) and the attention's parameters. */
typedef struct fk_attend_args {
  uint64_t q;        /* f32 [heads * head_dim]: the row's queries, before RoPE */
  uint64_t knew;     /* f32 [kv_heads * head_dim]: the new key row (read when p.store) */
  uint64_t vnew;     /* f32 [kv_heads * head_dim]: the new value row (read when p.store) */
  uint64_t kc;       /* f16 or bf16 [slots][kv_heads][length][head_dim]: the key ring */
  uint64_t vc;       /* the value ring, the same layout */
  uint64_t position; /* u32 [1] */
  uint64_t slot;     /* u32 [1] */
  uint64_t rope;     /* f32 [rope_rows][rotated][2]: cosines and sines (read when p.rope or p.krope) */
  uint64_t out;      /* f32 [heads * head_dim]: the attention's rows */
  fk_step_attend_params p; /* p.splits: ceil(length / p.split) */
} fk_attend_args;

/* The attention step; its splits' partial results go to a workspace the
 * context allocates (hipMalloc) on first use and grows when a call needs
 * more, which it refuses (FK_ERR_STATE) on a stream being captured.  The
 * context has one workspace: calls from several threads are serialized
 * while they grow it and queue their launches, but calls on one context
 * whose work overlaps on the GPU (two fk_streams, or a stream's work still
 * running when another's is queued) race on the same partials; such callers
 * order their streams, or take one context each.
 * Source: src/FuryKernel/Program/Eval.hs:474-527 (Attend), Plan.hs:174-181
 * (Partials + Combine). */
int fk_attend_decode(fk_ctx *ctx, const fk_attend_args *args, fk_stream *stream);

/* The most bytes of partial results fk_attend_decode_noalloc takes:
 * heads * splits * (head_dim + 2) * 4 must not exceed it (4 MiB; the 1B
 * decode's 32 heads x 32 splits x 66 x 4 is 270,336). */
#define FK_ATTEND_SCRATCH_BYTES (4u << 20)

/* fk_attend_decode with no allocation at all: its partial results go to a
 * static device array of FK_ATTEND_SCRATCH_BYTES that the library holds on
 * each GPU until the process ends (its address looked up at fk_init).  No
 * counterpart in the reference: for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * A larger step is refused with FK_ERR_RANGE.  Every call on a GPU shares that
 * GPU's array and each call overwrites the partials it reads (nothing needs
 * clearing): calls that overlap on one GPU (two streams, two contexts) race. */
int fk_attend_decode_noalloc(fk_ctx *ctx, const fk_attend_args *args, fk_stream *stream);

#ifdef __cplusplus
}
#endif

#endif /* FKROCM_OPS_H */
