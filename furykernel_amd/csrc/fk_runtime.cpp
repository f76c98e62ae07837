// fk_runtime.cpp — the C ABI of include/fkrocm.h over the HIP runtime.
//
// A thin shim: every entry point checks its handles and sizes, makes one or a
// few HIP calls, and turns a failure into a status and a message kept on the
// context (the reference's errors are values: src/FuryKernel/Interp.hs:148-186).
// Kernels come from code objects loaded with hipModuleLoadData and are launched
// with their kernarg bytes, as a LoweredKernel's launch table describes them
// (src/FuryKernel/Backend.hs:76-101).

#include "../../include/fkrocm.h"

#include <hip/hip_runtime_api.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "fk_internal.h"

namespace {

thread_local std::string g_init_error;

int fail(fk_ctx *ctx, int code, const char *fmt, ...) {
  char msg[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  if (ctx) {
    ctx->last_error = msg;
  } else {
    g_init_error = msg;
  }
  return code;
}

int hip_fail(fk_ctx *ctx, hipError_t e, const char *what) {
  return fail(ctx, FK_ERR_HIP, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

#define FK_HIP(ctx, call)                       \
  do {                                          \
    hipError_t fk_e_ = (call);                  \
    if (fk_e_ != hipSuccess) {                  \
      return hip_fail((ctx), fk_e_, #call);     \
    }                                           \
  } while (0)

hipStream_t stream_of(fk_ctx *ctx, fk_stream *s) { return s ? s->stream : ctx->stream; }

bool power_of_two(size_t a) { return a != 0 && (a & (a - 1)) == 0; }

// Makes the context's device current on this thread: HIP keeps the current
// device per thread, and a context may be driven from several.
int use_device(fk_ctx *ctx) {
  FK_HIP(ctx, hipSetDevice(ctx->device));
  return FK_OK;
}

}  // namespace

int fk_fail(fk_ctx *ctx, int code, const char *fmt, ...) {
  char msg[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  return fail(ctx, code, "%s", msg);
}

extern "C" {

int fk_init(int device, fk_ctx **out) {
  if (!out) return fail(nullptr, FK_ERR_ARG, "fk_init: null output");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return fail(nullptr, FK_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
  if (device < 0 || device >= count)
    return fail(nullptr, FK_ERR_RANGE, "fk_init: device %d of %d", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess) return fail(nullptr, FK_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  fk_ctx *ctx = new fk_ctx();
  ctx->device = device;
  // Default priority: streams of other priorities are not used.
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return fail(nullptr, FK_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  if (int st = fk_ops_setup(ctx)) {
    const std::string msg = ctx->last_error;
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(nullptr, st, "%s", msg.c_str());
  }
  *out = ctx;
  return FK_OK;
}

int fk_fini(fk_ctx *ctx) {
  if (!ctx) return fail(nullptr, FK_ERR_ARG, "fk_fini: null context");
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (fk_graph *g : ctx->graphs) {
    hipGraphExecDestroy(g->exec);
    hipGraphDestroy(g->graph);
    delete g;
  }
  for (fk_stream *s : ctx->streams) {
    hipStreamSynchronize(s->stream);
    hipStreamDestroy(s->stream);
    delete s;
  }
  for (fk_event *ev : ctx->events) {
    hipEventDestroy(ev->event);
    delete ev;
  }
  for (fk_buf *b : ctx->buffers) {
    if (!b->arena) hipFree(b->ptr);
    delete b;
  }
  for (fk_arena *a : ctx->arenas) {
    for (fk_buf *b : a->handed) delete b;
    hipFree(a->base);
    delete a;
  }
  for (fk_module *m : ctx->modules) {
    for (fk_fn *f : m->fns) delete f;
    hipModuleUnload(m->mod);
    delete m;
  }
  for (fk_table *t : ctx->tables) delete t;
  fk_ops_teardown(ctx);
  for (void *p : ctx->host) hipHostFree(p);
  hipStreamDestroy(ctx->stream);
  delete ctx;
  return FK_OK;
}

const char *fk_last_error(fk_ctx *ctx) { return ctx ? ctx->last_error.c_str() : g_init_error.c_str(); }

int fk_device_info_get(fk_ctx *ctx, fk_device_info *out) {
  if (!ctx || !out) return fail(ctx, FK_ERR_ARG, "fk_device_info_get: null argument");
  hipDeviceProp_t p;
  FK_HIP(ctx, hipGetDeviceProperties(&p, ctx->device));
  std::memset(out, 0, sizeof *out);
  std::snprintf(out->name, sizeof out->name, "%s", p.name);
  std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->simd_width = p.warpSize;
  out->max_threads = p.maxThreadsPerBlock;
  out->lds_bytes = static_cast<int32_t>(p.sharedMemPerBlock);
  out->global_bytes = static_cast<int64_t>(p.totalGlobalMem);
  out->l2_bytes = p.l2CacheSize;
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_bits = p.memoryBusWidth;
  return FK_OK;
}

// Modules -------------------------------------------------------------------

int fk_module_load(fk_ctx *ctx, const void *image, size_t bytes, fk_module **out) {
  if (!ctx || !image || !out || bytes == 0) return fail(ctx, FK_ERR_ARG, "fk_module_load: null or empty image");
  *out = nullptr;
  if (int s = use_device(ctx)) return s;
  hipModule_t mod;
  FK_HIP(ctx, hipModuleLoadData(&mod, image));
  fk_module *m = new fk_module{ctx, mod, {}};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->modules.insert(m);
  *out = m;
  return FK_OK;
}

int fk_module_load_file(fk_ctx *ctx, const char *path, fk_module **out) {
  if (!ctx || !path || !out) return fail(ctx, FK_ERR_ARG, "fk_module_load_file: null argument");
  std::ifstream f(path, std::ios::binary);
  if (!f) return fail(ctx, FK_ERR_NOT_FOUND, "fk_module_load_file: cannot open %s", path);
  std::vector<char> image((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (image.empty()) return fail(ctx, FK_ERR_ARG, "fk_module_load_file: %s is empty", path);
  return fk_module_load(ctx, image.data(), image.size(), out);
}

// hipRTC --------------------------------------------------------------------

int fk_rtc_compile(const char *source, const char *name, const char *const *options, int n_options, void **code,
                   size_t *code_bytes, char **log) {
  if (!source || !code || !code_bytes || n_options < 0 || (n_options > 0 && !options))
    return fail(nullptr, FK_ERR_ARG, "fk_rtc_compile: null argument");
  *code = nullptr;
  *code_bytes = 0;
  if (log) *log = nullptr;
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name ? name : "unit.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(nullptr, FK_ERR_COMPILE, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  r = hiprtcCompileProgram(prog, n_options, const_cast<const char **>(options));
  size_t log_bytes = 0;
  if (log && hiprtcGetProgramLogSize(prog, &log_bytes) == HIPRTC_SUCCESS && log_bytes > 1) {
    *log = static_cast<char *>(malloc(log_bytes + 1));
    if (*log) {
      hiprtcGetProgramLog(prog, *log);
      (*log)[log_bytes] = '\0';
    }
  }
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return fail(nullptr, FK_ERR_COMPILE, "fk_rtc_compile: %s: %s", name ? name : "unit.hip",
                hiprtcGetErrorString(r));
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  void *buf = n ? malloc(n) : nullptr;
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return fail(nullptr, FK_ERR_OOM, "fk_rtc_compile: no host memory for a code object of %zu bytes", n);
  }
  hiprtcGetCode(prog, static_cast<char *>(buf));
  hiprtcDestroyProgram(&prog);
  *code = buf;
  *code_bytes = n;
  return FK_OK;
}

void fk_rtc_free(void *p) { free(p); }

int fk_module_unload(fk_module *m) {
  if (!m) return fail(nullptr, FK_ERR_ARG, "fk_module_unload: null module");
  fk_ctx *ctx = m->ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->modules.erase(m);
  }
  for (fk_fn *f : m->fns) delete f;
  hipError_t e = hipModuleUnload(m->mod);
  delete m;
  if (e != hipSuccess) return hip_fail(ctx, e, "hipModuleUnload");
  return FK_OK;
}

int fk_function(fk_module *m, const char *entry, fk_fn **out) {
  if (!m || !entry || !out) return fail(m ? m->ctx : nullptr, FK_ERR_ARG, "fk_function: null argument");
  *out = nullptr;
  for (fk_fn *f : m->fns) {
    if (f->entry == entry) {
      *out = f;
      return FK_OK;
    }
  }
  hipFunction_t fn;
  hipError_t e = hipModuleGetFunction(&fn, m->mod, entry);
  if (e != hipSuccess) return fail(m->ctx, FK_ERR_NOT_FOUND, "fk_function: no entry %s (%s)", entry, hipGetErrorString(e));
  fk_fn *f = new fk_fn{m, fn, entry};
  m->fns.push_back(f);
  *out = f;
  return FK_OK;
}

// Memory --------------------------------------------------------------------

int fk_alloc(fk_ctx *ctx, size_t bytes, size_t align, fk_buf **out) {
  if (!ctx || !out) return fail(ctx, FK_ERR_ARG, "fk_alloc: null argument");
  *out = nullptr;
  if (bytes == 0) return fail(ctx, FK_ERR_ARG, "fk_alloc: zero bytes");
  if (!power_of_two(align) || align > 4096)
    return fail(ctx, FK_ERR_ARG, "fk_alloc: alignment %zu is not a power of two up to 4096", align);
  if (int s = use_device(ctx)) return s;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);  // 4096-aligned at least
  if (e == hipErrorOutOfMemory) return fail(ctx, FK_ERR_OOM, "fk_alloc: %zu bytes: out of device memory", bytes);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc");
  fk_buf *b = new fk_buf{ctx, nullptr, p, bytes};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->buffers.insert(b);
  *out = b;
  return FK_OK;
}

int fk_free(fk_buf *b) {
  if (!b) return fail(nullptr, FK_ERR_ARG, "fk_free: null buffer");
  fk_ctx *ctx = b->ctx;
  if (b->arena) return fail(ctx, FK_ERR_STATE, "fk_free: an arena's buffer is freed with its arena");
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->buffers.erase(b);
  }
  hipError_t e = hipFree(b->ptr);
  delete b;
  if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
  return FK_OK;
}

uint64_t fk_buf_ptr(const fk_buf *b) { return b ? reinterpret_cast<uint64_t>(b->ptr) : 0; }

size_t fk_buf_size(const fk_buf *b) { return b ? b->size : 0; }

int fk_arena_create(fk_ctx *ctx, size_t bytes, fk_arena **out) {
  if (!ctx || !out || bytes == 0) return fail(ctx, FK_ERR_ARG, "fk_arena_create: null argument or zero bytes");
  *out = nullptr;
  if (int s = use_device(ctx)) return s;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e == hipErrorOutOfMemory) return fail(ctx, FK_ERR_OOM, "fk_arena_create: %zu bytes: out of device memory", bytes);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc");
  fk_arena *a = new fk_arena{ctx, p, bytes, 0, {}};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->arenas.insert(a);
  *out = a;
  return FK_OK;
}

int fk_arena_destroy(fk_arena *a) {
  if (!a) return fail(nullptr, FK_ERR_ARG, "fk_arena_destroy: null arena");
  fk_ctx *ctx = a->ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->arenas.erase(a);
  }
  for (fk_buf *b : a->handed) delete b;
  hipError_t e = hipFree(a->base);
  delete a;
  if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
  return FK_OK;
}

int fk_arena_alloc(fk_arena *a, size_t bytes, size_t align, fk_buf **out) {
  if (!a || !out) return fail(a ? a->ctx : nullptr, FK_ERR_ARG, "fk_arena_alloc: null argument");
  *out = nullptr;
  if (bytes == 0) return fail(a->ctx, FK_ERR_ARG, "fk_arena_alloc: zero bytes");
  if (!power_of_two(align) || align < 16 || align > 4096)
    return fail(a->ctx, FK_ERR_ARG, "fk_arena_alloc: alignment %zu is not a power of two in [16, 4096]", align);
  size_t at = (a->used + align - 1) & ~(align - 1);
  if (at > a->capacity || bytes > a->capacity - at)
    return fail(a->ctx, FK_ERR_OOM, "fk_arena_alloc: %zu bytes at %zu exceed the arena's %zu", bytes, at, a->capacity);
  fk_buf *b = new fk_buf{a->ctx, a, static_cast<char *>(a->base) + at, bytes};
  a->used = at + bytes;
  a->handed.push_back(b);
  *out = b;
  return FK_OK;
}

int fk_arena_usage(const fk_arena *a, size_t *used, size_t *capacity) {
  if (!a || !used || !capacity) return fail(a ? a->ctx : nullptr, FK_ERR_ARG, "fk_arena_usage: null argument");
  *used = a->used;
  *capacity = a->capacity;
  return FK_OK;
}

int fk_arena_reset(fk_arena *a) {
  if (!a) return fail(nullptr, FK_ERR_ARG, "fk_arena_reset: null arena");
  for (fk_buf *b : a->handed) delete b;
  a->handed.clear();
  a->used = 0;
  return FK_OK;
}

int fk_host_alloc(fk_ctx *ctx, size_t bytes, void **out) {
  if (!ctx || !out || bytes == 0) return fail(ctx, FK_ERR_ARG, "fk_host_alloc: null argument or zero bytes");
  *out = nullptr;
  if (int s = use_device(ctx)) return s;
  void *p = nullptr;
  FK_HIP(ctx, hipHostMalloc(&p, bytes, hipHostMallocDefault));
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->host.insert(p);
  *out = p;
  return FK_OK;
}

int fk_host_free(fk_ctx *ctx, void *p) {
  if (!ctx || !p) return fail(ctx, FK_ERR_ARG, "fk_host_free: null argument");
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (!ctx->host.erase(p)) return fail(ctx, FK_ERR_ARG, "fk_host_free: not this context's pinned memory");
  }
  FK_HIP(ctx, hipHostFree(p));
  return FK_OK;
}

static int check_span(fk_ctx *ctx, const fk_buf *b, size_t off, size_t bytes, const char *what) {
  if (!b) return fail(ctx, FK_ERR_ARG, "%s: null buffer", what);
  if (off > b->size || bytes > b->size - off)
    return fail(ctx, FK_ERR_RANGE, "%s: %zu bytes at %zu of a buffer of %zu", what, bytes, off, b->size);
  return FK_OK;
}

int fk_copy_h2d_async(fk_ctx *ctx, fk_buf *dst, size_t off, const void *src, size_t bytes, fk_stream *s) {
  if (!ctx || (!src && bytes)) return fail(ctx, FK_ERR_ARG, "fk_copy_h2d_async: null argument");
  if (int st = check_span(ctx, dst, off, bytes, "fk_copy_h2d_async")) return st;
  if (bytes == 0) return FK_OK;
  FK_HIP(ctx, hipMemcpyAsync(static_cast<char *>(dst->ptr) + off, src, bytes, hipMemcpyHostToDevice, stream_of(ctx, s)));
  return FK_OK;
}

int fk_copy_d2h_async(fk_ctx *ctx, void *dst, const fk_buf *src, size_t off, size_t bytes, fk_stream *s) {
  if (!ctx || (!dst && bytes)) return fail(ctx, FK_ERR_ARG, "fk_copy_d2h_async: null argument");
  if (int st = check_span(ctx, src, off, bytes, "fk_copy_d2h_async")) return st;
  if (bytes == 0) return FK_OK;
  FK_HIP(ctx, hipMemcpyAsync(dst, static_cast<const char *>(src->ptr) + off, bytes, hipMemcpyDeviceToHost, stream_of(ctx, s)));
  return FK_OK;
}

int fk_copy_d2d_async(fk_ctx *ctx, fk_buf *dst, size_t doff, const fk_buf *src, size_t soff, size_t bytes, fk_stream *s) {
  if (!ctx) return fail(ctx, FK_ERR_ARG, "fk_copy_d2d_async: null context");
  if (int st = check_span(ctx, dst, doff, bytes, "fk_copy_d2d_async (destination)")) return st;
  if (int st = check_span(ctx, src, soff, bytes, "fk_copy_d2d_async (source)")) return st;
  if (bytes == 0) return FK_OK;
  FK_HIP(ctx, hipMemcpyAsync(static_cast<char *>(dst->ptr) + doff, static_cast<const char *>(src->ptr) + soff, bytes,
                             hipMemcpyDeviceToDevice, stream_of(ctx, s)));
  return FK_OK;
}

int fk_memset_async(fk_ctx *ctx, fk_buf *dst, size_t off, int value, size_t bytes, fk_stream *s) {
  if (!ctx) return fail(ctx, FK_ERR_ARG, "fk_memset_async: null context");
  if (int st = check_span(ctx, dst, off, bytes, "fk_memset_async")) return st;
  if (bytes == 0) return FK_OK;
  // A memset node in a captured graph has given wrong results on replays
  // after the first on this platform: a graph clears memory with a kernel.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  FK_HIP(ctx, hipStreamIsCapturing(stream_of(ctx, s), &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(ctx, FK_ERR_STATE, "fk_memset_async: the stream is being captured; clear memory with a kernel");
  FK_HIP(ctx, hipMemsetAsync(static_cast<char *>(dst->ptr) + off, value, bytes, stream_of(ctx, s)));
  return FK_OK;
}

// Streams -------------------------------------------------------------------

int fk_stream_create(fk_ctx *ctx, fk_stream **out) {
  if (!ctx || !out) return fail(ctx, FK_ERR_ARG, "fk_stream_create: null argument");
  *out = nullptr;
  if (int s = use_device(ctx)) return s;
  hipStream_t st;
  FK_HIP(ctx, hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  fk_stream *s = new fk_stream{ctx, st};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->streams.insert(s);
  *out = s;
  return FK_OK;
}

int fk_stream_destroy(fk_stream *s) {
  if (!s) return fail(nullptr, FK_ERR_ARG, "fk_stream_destroy: null stream");
  fk_ctx *ctx = s->ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->streams.erase(s);
  }
  hipStreamSynchronize(s->stream);
  hipError_t e = hipStreamDestroy(s->stream);
  delete s;
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamDestroy");
  return FK_OK;
}

int fk_stream_sync(fk_ctx *ctx, fk_stream *s) {
  if (!ctx) return fail(ctx, FK_ERR_ARG, "fk_stream_sync: null context");
  FK_HIP(ctx, hipStreamSynchronize(stream_of(ctx, s)));
  return FK_OK;
}

// Launch --------------------------------------------------------------------

int fk_launch(fk_fn *fn, uint32_t groups, uint32_t threads, uint32_t lds_bytes, const void *kernarg,
              size_t kernarg_bytes, fk_stream *s) {
  if (!fn) return fail(nullptr, FK_ERR_ARG, "fk_launch: null function");
  fk_ctx *ctx = fn->mod->ctx;
  if (groups == 0) return FK_OK;
  if (threads == 0 || threads > 1024)
    return fail(ctx, FK_ERR_RANGE, "fk_launch %s: %u threads per group, not 1 to 1024", fn->entry.c_str(), threads);
  if (lds_bytes > 160 * 1024)
    return fail(ctx, FK_ERR_RANGE, "fk_launch %s: %u bytes of threadgroup memory, more than 160 KiB", fn->entry.c_str(), lds_bytes);
  if (!kernarg && kernarg_bytes) return fail(ctx, FK_ERR_ARG, "fk_launch %s: null kernarg", fn->entry.c_str());
  // hipModuleLaunchKernel copies the kernarg bytes at the call.
  size_t size = kernarg_bytes;
  void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void *>(kernarg), HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(fn->fn, groups, 1, 1, threads, 1, 1, lds_bytes, stream_of(ctx, s), nullptr,
                                       kernarg_bytes ? config : nullptr);
  if (e != hipSuccess) return fail(ctx, FK_ERR_HIP, "fk_launch %s: %s", fn->entry.c_str(), hipGetErrorString(e));
  return FK_OK;
}

// Launch tables ---------------------------------------------------------------

int fk_table_create(fk_ctx *ctx, fk_table **out) {
  if (!ctx || !out) return fail(ctx, FK_ERR_ARG, "fk_table_create: null argument");
  fk_table *t = new fk_table{ctx, {}};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->tables.insert(t);
  *out = t;
  return FK_OK;
}

int fk_table_destroy(fk_table *t) {
  if (!t) return fail(nullptr, FK_ERR_ARG, "fk_table_destroy: null table");
  {
    std::lock_guard<std::mutex> lock(t->ctx->mu);
    t->ctx->tables.erase(t);
  }
  delete t;
  return FK_OK;
}

int fk_table_add(fk_table *t, fk_fn *fn, uint32_t groups, uint32_t threads, uint32_t lds_bytes,
                 const fk_binding *buffers, uint32_t n_buffers, const void *params, size_t params_bytes,
                 uint64_t abi_hash, uint32_t *index) {
  if (!t || !fn) return fail(t ? t->ctx : nullptr, FK_ERR_ARG, "fk_table_add: null table or function");
  char err[512];
  const int st = fk_launch_check(fn->entry.c_str(), groups, threads, lds_bytes, buffers, n_buffers, params,
                                 params_bytes, abi_hash, err, sizeof err);
  if (st != FK_OK) return fail(t->ctx, st, "fk_table_add: %s", err);
  fk_table::Launch l{fn, groups, threads, lds_bytes, {}};
  l.kernarg.resize(8 * (size_t)n_buffers + params_bytes);
  for (uint32_t i = 0; i < n_buffers; i++) std::memcpy(l.kernarg.data() + 8 * i, &buffers[i].addr, 8);
  if (params_bytes) std::memcpy(l.kernarg.data() + 8 * (size_t)n_buffers, params, params_bytes);
  t->launches.push_back(std::move(l));
  if (index) *index = (uint32_t)(t->launches.size() - 1);
  return FK_OK;
}

int fk_table_count(const fk_table *t, uint32_t *count) {
  if (!t || !count) return fail(t ? t->ctx : nullptr, FK_ERR_ARG, "fk_table_count: null argument");
  *count = (uint32_t)t->launches.size();
  return FK_OK;
}

int fk_table_enqueue(fk_table *t, uint32_t first, uint32_t count, fk_stream *s) {
  if (!t) return fail(nullptr, FK_ERR_ARG, "fk_table_enqueue: null table");
  if (first > t->launches.size() || count > t->launches.size() - first)
    return fail(t->ctx, FK_ERR_RANGE, "fk_table_enqueue: launches [%u, %u) of %zu", first, first + count,
                t->launches.size());
  for (uint32_t i = first; i < first + count; i++) {
    const fk_table::Launch &l = t->launches[i];
    if (int st = fk_launch(l.fn, l.groups, l.threads, l.lds_bytes, l.kernarg.data(), l.kernarg.size(), s)) return st;
  }
  return FK_OK;
}

// Events --------------------------------------------------------------------

int fk_event_create(fk_ctx *ctx, fk_event **out) {
  if (!ctx || !out) return fail(ctx, FK_ERR_ARG, "fk_event_create: null argument");
  *out = nullptr;
  if (int s = use_device(ctx)) return s;
  hipEvent_t ev;
  FK_HIP(ctx, hipEventCreate(&ev));
  fk_event *e = new fk_event{ctx, ev};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->events.insert(e);
  *out = e;
  return FK_OK;
}

int fk_event_destroy(fk_event *e) {
  if (!e) return fail(nullptr, FK_ERR_ARG, "fk_event_destroy: null event");
  fk_ctx *ctx = e->ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->events.erase(e);
  }
  hipError_t err = hipEventDestroy(e->event);
  delete e;
  if (err != hipSuccess) return hip_fail(ctx, err, "hipEventDestroy");
  return FK_OK;
}

int fk_event_record(fk_event *e, fk_stream *s) {
  if (!e) return fail(nullptr, FK_ERR_ARG, "fk_event_record: null event");
  FK_HIP(e->ctx, hipEventRecord(e->event, stream_of(e->ctx, s)));
  return FK_OK;
}

int fk_event_sync(fk_event *e) {
  if (!e) return fail(nullptr, FK_ERR_ARG, "fk_event_sync: null event");
  FK_HIP(e->ctx, hipEventSynchronize(e->event));
  return FK_OK;
}

int fk_stream_wait_event(fk_stream *s, fk_event *e) {
  if (!e) return fail(nullptr, FK_ERR_ARG, "fk_stream_wait_event: null event");
  FK_HIP(e->ctx, hipStreamWaitEvent(stream_of(e->ctx, s), e->event, 0));
  return FK_OK;
}

int fk_event_elapsed_ms(fk_event *a, fk_event *b, float *ms) {
  if (!a || !b || !ms) return fail(a ? a->ctx : nullptr, FK_ERR_ARG, "fk_event_elapsed_ms: null argument");
  FK_HIP(a->ctx, hipEventElapsedTime(ms, a->event, b->event));
  return FK_OK;
}

// Graphs --------------------------------------------------------------------

int fk_graph_begin(fk_ctx *ctx, fk_stream *s) {
  if (!ctx) return fail(ctx, FK_ERR_ARG, "fk_graph_begin: null context");
  FK_HIP(ctx, hipStreamBeginCapture(stream_of(ctx, s), hipStreamCaptureModeThreadLocal));
  return FK_OK;
}

int fk_graph_end(fk_ctx *ctx, fk_stream *s, fk_graph **out) {
  if (!ctx || !out) return fail(ctx, FK_ERR_ARG, "fk_graph_end: null argument");
  *out = nullptr;
  hipGraph_t g;
  hipError_t e = hipStreamEndCapture(stream_of(ctx, s), &g);
  if (e == hipErrorIllegalState) return fail(ctx, FK_ERR_STATE, "fk_graph_end: the stream is not capturing");
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
  hipGraphExec_t exec;
  e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g);
    return hip_fail(ctx, e, "hipGraphInstantiate");
  }
  fk_graph *gr = new fk_graph{ctx, g, exec};
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->graphs.insert(gr);
  *out = gr;
  return FK_OK;
}

int fk_graph_replay(fk_graph *g, fk_stream *s) {
  if (!g) return fail(nullptr, FK_ERR_ARG, "fk_graph_replay: null graph");
  FK_HIP(g->ctx, hipGraphLaunch(g->exec, stream_of(g->ctx, s)));
  return FK_OK;
}

int fk_graph_destroy(fk_graph *g) {
  if (!g) return fail(nullptr, FK_ERR_ARG, "fk_graph_destroy: null graph");
  fk_ctx *ctx = g->ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->graphs.erase(g);
  }
  hipGraphExecDestroy(g->exec);
  hipError_t e = hipGraphDestroy(g->graph);
  delete g;
  if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphDestroy");
  return FK_OK;
}

}  // extern "C"
