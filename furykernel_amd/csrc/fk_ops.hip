// fk_ops.hip — whole operations as one C call (include/fkrocm_ops.h): the
// decode attention step over a ring KV cache, with the same device code as
// the planned step's attention and combine launches (kernels/fk_attention.h),
// compiled into the C ABI's library.

#include "../../include/fkrocm_ops.h"

#include <hip/hip_runtime.h>

#include <mutex>

#include "fk_internal.h"
#include "kernels/fk_attention.h"

namespace {

__global__ void __launch_bounds__(FK_ATTN_THREADS)
    op_attend(const float *__restrict__ q, const float *__restrict__ knew, const float *__restrict__ vnew,
              uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const uint32_t *__restrict__ position,
              const uint32_t *__restrict__ slot, const float *__restrict__ rope, float *__restrict__ partials,
              fk_step_attend_params p) {
  fk::step_attend(q, knew, vnew, kc, vc, position, slot, rope, partials, position, p);
}

__global__ void __launch_bounds__(FK_WAVE)
    op_combine(const float *__restrict__ partials, float *__restrict__ out, fk_step_combine_params p) {
  fk::step_combine(partials, out, p);
}

// The bytes of partial results a step makes, after checking its arguments
// against what the kernels take (0 and a message on the context if not).
size_t check_attend(fk_ctx *ctx, const fk_attend_args *a, const char *what) {
  const fk_step_attend_params &p = a->p;
  if (p.has_reach) {
    fk_fail(ctx, FK_ERR_ARG, "%s: the one-call attention takes no reach", what);
    return 0;
  }
  if (p.kv_heads == 0 || p.heads % p.kv_heads || p.heads / p.kv_heads > 8 || p.head_dim == 0 || p.head_dim > 64 ||
      p.head_dim % 8 || (p.split != 64 && p.split != 128) || p.length == 0 || p.slots == 0 ||
      p.splits != (p.length + p.split - 1) / p.split) {
    fk_fail(ctx, FK_ERR_ARG, "%s: %u heads over %u of width %u, splits of %u, %u splits of a ring of %u", what,
            p.heads, p.kv_heads, p.head_dim, p.split, p.splits, p.length);
    return 0;
  }
  if ((p.rope || p.krope) && (p.rotated == 0 || 2 * p.rotated > p.head_dim || p.rope_rows == 0 || !a->rope)) {
    fk_fail(ctx, FK_ERR_ARG, "%s: RoPE of %u pairs of a head of %u from a table of %u rows", what, p.rotated,
            p.head_dim, p.rope_rows);
    return 0;
  }
  const uint64_t need[] = {a->q, a->kc, a->vc, a->position, a->slot, a->out};
  for (uint64_t x : need)
    if (x == 0 || x % 16) {
      fk_fail(ctx, FK_ERR_ARG, "%s: a null or misaligned buffer", what);
      return 0;
    }
  if (p.store && (a->knew == 0 || a->vnew == 0 || a->knew % 16 || a->vnew % 16)) {
    fk_fail(ctx, FK_ERR_ARG, "%s: a store without its new rows", what);
    return 0;
  }
  return (size_t)p.heads * p.splits * (p.head_dim + 2) * sizeof(float);
}

int launch_attend(fk_ctx *ctx, const fk_attend_args *a, float *partials, hipStream_t s, const char *what) {
  const fk_step_attend_params &p = a->p;
  hipLaunchKernelGGL(op_attend, dim3(p.kv_heads * p.splits), dim3(FK_ATTN_THREADS), 0, s,
                     reinterpret_cast<const float *>(a->q), reinterpret_cast<const float *>(a->knew),
                     reinterpret_cast<const float *>(a->vnew), reinterpret_cast<uint16_t *>(a->kc),
                     reinterpret_cast<uint16_t *>(a->vc), reinterpret_cast<const uint32_t *>(a->position),
                     reinterpret_cast<const uint32_t *>(a->slot),
                     reinterpret_cast<const float *>(a->rope ? a->rope : a->position), partials, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fk_fail(ctx, FK_ERR_HIP, "%s (attention): %s", what, hipGetErrorString(e));
  const fk_step_combine_params c = {p.heads, p.head_dim, p.splits};
  hipLaunchKernelGGL(op_combine, dim3(p.heads), dim3(FK_WAVE), 0, s, partials, reinterpret_cast<float *>(a->out), c);
  e = hipGetLastError();
  if (e != hipSuccess) return fk_fail(ctx, FK_ERR_HIP, "%s (combine): %s", what, hipGetErrorString(e));
  return FK_OK;
}

// fk_attend_decode_noalloc's partial results: one static array on each GPU,
// held until the process ends.  In host code `scratch` names a host-side
// stand-in, not a device address: only the address hipGetSymbolAddress gives
// for a device (kept per device below) is passed to kernels.
__device__ __align__(256) float scratch[FK_ATTEND_SCRATCH_BYTES / sizeof(float)];

std::mutex g_scratch_mu;
void *g_scratch[64];  // by device ordinal

}  // namespace

// At fk_init, with the context's device current: the static scratch's address
// on that device, looked up once per device.
int fk_ops_setup(fk_ctx *ctx) {
  if (ctx->device < 0 || ctx->device >= 64)
    return fk_fail(ctx, FK_ERR_RANGE, "fk_init: device %d past the 64 the operations track", ctx->device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[ctx->device]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fk_fail(ctx, FK_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", ctx->device,
                     hipGetErrorString(e));
    g_scratch[ctx->device] = ptr;
  }
  ctx->scratch = g_scratch[ctx->device];
  return FK_OK;
}

void fk_ops_teardown(fk_ctx *ctx) {
  if (ctx->workspace) {
    hipFree(ctx->workspace);
    ctx->workspace = nullptr;
    ctx->workspace_bytes = 0;
  }
}

extern "C" int fk_attend_decode(fk_ctx *ctx, const fk_attend_args *a, fk_stream *stream) {
  if (!ctx || !a) return fk_fail(ctx, FK_ERR_ARG, "fk_attend_decode: null argument");
  const size_t bytes = check_attend(ctx, a, "fk_attend_decode");
  if (bytes == 0) return FK_ERR_ARG;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return fk_fail(ctx, FK_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  hipStream_t s = stream ? stream->stream : ctx->stream;
  std::lock_guard<std::mutex> lock(ctx->workspace_mu);
  if (bytes > ctx->workspace_bytes) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(s, &cap);
    if (e != hipSuccess) return fk_fail(ctx, FK_ERR_HIP, "hipStreamIsCapturing: %s", hipGetErrorString(e));
    if (cap != hipStreamCaptureStatusNone)
      return fk_fail(ctx, FK_ERR_STATE, "fk_attend_decode: the workspace must grow to %zu bytes while the stream is "
                     "captured; call it once before capturing", bytes);
    // Work queued before on any stream may still read the old workspace.
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return fk_fail(ctx, FK_ERR_HIP, "hipDeviceSynchronize: %s", hipGetErrorString(e));
    if (ctx->workspace) hipFree(ctx->workspace);
    ctx->workspace = nullptr;
    ctx->workspace_bytes = 0;
    e = hipMalloc(&ctx->workspace, bytes);
    if (e != hipSuccess) return fk_fail(ctx, FK_ERR_OOM, "fk_attend_decode: a workspace of %zu bytes: %s", bytes,
                                        hipGetErrorString(e));
    ctx->workspace_bytes = bytes;
  }
  return launch_attend(ctx, a, static_cast<float *>(ctx->workspace), s, "fk_attend_decode");
}

extern "C" int fk_attend_decode_noalloc(fk_ctx *ctx, const fk_attend_args *a, fk_stream *stream) {
  if (!ctx || !a) return fk_fail(ctx, FK_ERR_ARG, "fk_attend_decode_noalloc: null argument");
  const size_t bytes = check_attend(ctx, a, "fk_attend_decode_noalloc");
  if (bytes == 0) return FK_ERR_ARG;
  if (bytes > FK_ATTEND_SCRATCH_BYTES)
    return fk_fail(ctx, FK_ERR_RANGE,
                   "fk_attend_decode_noalloc: %zu bytes of partial results (heads %u x splits %u x (head_dim %u + 2) "
                   "x 4); the static scratch holds %u",
                   bytes, a->p.heads, a->p.splits, a->p.head_dim, FK_ATTEND_SCRATCH_BYTES);
  if (!ctx->scratch) return fk_fail(ctx, FK_ERR_STATE, "fk_attend_decode_noalloc: no scratch on this device");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return fk_fail(ctx, FK_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  return launch_attend(ctx, a, static_cast<float *>(ctx->scratch), stream ? stream->stream : ctx->stream,
                       "fk_attend_decode_noalloc");
}
