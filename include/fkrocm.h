/*
 * fkrocm.h — the C ABI of FuryKernel's MI355X (gfx950) execution target.
 *
 * This is the FFI surface a `FuryKernel.Rocm` target library binds with
 * `foreign import ccall`: the runtime a `Backend Rocm`'s launch tables run
 * on.  It replaces, for the ROCm target, what the CPU target does in-process
 * (src/FuryKernel/Cpu.hs:271-278: a kernel is a function of its parameter
 * struct's bytes, its buffers and its tables) and what a GPU runtime must do
 * for a `LoweredKernel` (src/FuryKernel/Backend.hs:76-101): load the
 * translation unit, bind buffers in `lkBindings` order, pass the parameter
 * struct in C layout (src/FuryKernel/Abi.hs:113-133), launch `lkGroups`
 * threadgroups of `lkThreads` threads with `lkTgMemory` bytes of threadgroup
 * memory, and skip a launch of zero groups (src/FuryKernel/Backend.hs:84-87).
 *
 * Conventions
 *  - Every call returns an `int` status: FK_OK (0) or a negative FK_ERR_*.
 *    The context keeps the message of its last failure (`fk_last_error`),
 *    as the reference's errors are values (src/FuryKernel/Interp.hs:148-186).
 *  - Ownership: a context owns device memory, modules, streams, events and
 *    graphs made through it; the caller owns host memory.  Kernarg bytes are
 *    copied at launch, so the caller may reuse them at once.
 *  - Threading: one context per device.  Calls on one stream are ordered;
 *    distinct streams may be driven from distinct threads.
 *  - A NULL `fk_stream*` means the context's own stream.
 *  - No pointers of other libraries' types cross this ABI: buffers are
 *    handles, device addresses are `uint64_t`, sizes are `size_t`.
 */
#ifndef FKROCM_H
#define FKROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  FK_OK = 0,
  FK_ERR_HIP = -1,       /* the HIP runtime refused a call */
  FK_ERR_ARG = -2,       /* a null handle, a bad size, a bad alignment */
  FK_ERR_RANGE = -3,     /* a copy or launch outside what was allocated or allowed */
  FK_ERR_NOT_FOUND = -4, /* an entry point the module lacks, a missing file */
  FK_ERR_STATE = -5,     /* a call out of order (graph capture not begun, ...) */
  FK_ERR_OOM = -6,       /* device or arena memory exhausted */
  FK_ERR_COMPILE = -7    /* hipRTC refused a translation unit (fk_rtc_compile's log says why) */
};

typedef struct fk_ctx fk_ctx;
typedef struct fk_module fk_module;
typedef struct fk_fn fk_fn;
typedef struct fk_buf fk_buf;
typedef struct fk_arena fk_arena;
typedef struct fk_stream fk_stream;
typedef struct fk_event fk_event;
typedef struct fk_graph fk_graph;

/* What the device is: the reflected caps of `instance Target Rocm`
 * (src/FuryKernel/Target.hs:73-98) plus what tuning needs. */
typedef struct fk_device_info {
  char name[256];           /* marketing name */
  char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;    /* CUs (the tuning Profile's cores) */
  int32_t simd_width;       /* lanes per SIMD group (wavefront) */
  int32_t max_threads;      /* threads per threadgroup */
  int32_t lds_bytes;        /* threadgroup memory per threadgroup */
  int64_t global_bytes;     /* HBM */
  int32_t l2_bytes;         /* L2 per XCD as the runtime reports it */
  int32_t clock_khz;        /* peak shader clock */
  int32_t memory_clock_khz; /* peak memory clock */
  int32_t memory_bus_bits;  /* memory bus width */
} fk_device_info;

/* Context. ---------------------------------------------------------------- */

/* Opens device `device` and makes its stream. */
int fk_init(int device, fk_ctx **out);
/* Frees everything the context made, then the context. */
int fk_fini(fk_ctx *ctx);
/* The message of the context's last failure ("" if none); valid until the
 * next call on the context.  With a NULL context, the last failure of
 * fk_init on this thread. */
const char *fk_last_error(fk_ctx *ctx);
int fk_device_info_get(fk_ctx *ctx, fk_device_info *out);

/* Modules: a code object (hsaco) with the kernels of one translation unit
 * (the `Lowered`'s `loweredSource`, compiled). ------------------------------ */

int fk_module_load(fk_ctx *ctx, const void *image, size_t bytes, fk_module **out);
int fk_module_load_file(fk_ctx *ctx, const char *path, fk_module **out);
int fk_module_unload(fk_module *mod);
/* The kernel `entry` (a `LoweredKernel`'s `lkEntry`). */
int fk_function(fk_module *mod, const char *entry, fk_fn **out);

/* hipRTC: a lowered translation unit's HIP source (the `Lowered`'s
 * `loweredSource`, src/FuryKernel/Backend.hs:37-44, as the IR target of
 * furykernel_amd/ir/rocm.py emits it) compiled for the device at run time, as
 * the reference's runtimes compile a backend's source (Backend.hs:4-11).
 * Needs no device or context.  On success `*code` is a code object of
 * `*code_bytes` for fk_module_load; on FK_ERR_COMPILE, `*log` (if `log` is
 * given) holds the compiler's messages.  Both are the caller's to free with
 * fk_rtc_free.  Failures are reported by fk_last_error(NULL). */
int fk_rtc_compile(const char *source, const char *name, const char *const *options, int n_options, void **code,
                   size_t *code_bytes, char **log);
void fk_rtc_free(void *p);

/* Device memory. -------------------------------------------------------------
 * A buffer is a handle on device memory with its size; its device address is
 * what kernargs carry.  `fk_alloc` takes memory of its own; an arena takes
 * one allocation up front and carves resident buffers out of it (weights,
 * KV caches, the values steps store), which live until the arena is reset
 * or destroyed. */

int fk_alloc(fk_ctx *ctx, size_t bytes, size_t align, fk_buf **out);
int fk_free(fk_buf *buf);
uint64_t fk_buf_ptr(const fk_buf *buf);
size_t fk_buf_size(const fk_buf *buf);

int fk_arena_create(fk_ctx *ctx, size_t bytes, fk_arena **out);
int fk_arena_destroy(fk_arena *arena);
/* A buffer of `bytes` at a multiple of `align` (a power of two, at least 16,
 * as Type.hs:70-71's leastAlign has it) inside the arena. */
int fk_arena_alloc(fk_arena *arena, size_t bytes, size_t align, fk_buf **out);
/* Bytes handed out so far, and the arena's capacity. */
int fk_arena_usage(const fk_arena *arena, size_t *used, size_t *capacity);
/* Forgets every buffer the arena handed out (their handles become invalid). */
int fk_arena_reset(fk_arena *arena);

/* Pinned host memory, for copies that overlap work. */
int fk_host_alloc(fk_ctx *ctx, size_t bytes, void **out);
int fk_host_free(fk_ctx *ctx, void *ptr);

/* Copies, ordered on the stream.  Offsets and sizes in bytes, checked
 * against the buffers' sizes (FK_ERR_RANGE). */
int fk_copy_h2d_async(fk_ctx *ctx, fk_buf *dst, size_t dst_offset, const void *src, size_t bytes,
                      fk_stream *stream);
int fk_copy_d2h_async(fk_ctx *ctx, void *dst, const fk_buf *src, size_t src_offset, size_t bytes,
                      fk_stream *stream);
int fk_copy_d2d_async(fk_ctx *ctx, fk_buf *dst, size_t dst_offset, const fk_buf *src,
                      size_t src_offset, size_t bytes, fk_stream *stream);
/* Sets `bytes` bytes to `value`.  Not for code a graph captures: on a stream
 * being captured it returns FK_ERR_STATE, and a graph clears memory with a
 * kernel of the module instead. */
int fk_memset_async(fk_ctx *ctx, fk_buf *dst, size_t dst_offset, int value, size_t bytes,
                    fk_stream *stream);

/* Streams (default priority only). */
int fk_stream_create(fk_ctx *ctx, fk_stream **out);
int fk_stream_destroy(fk_stream *stream);
/* Waits for everything queued on the stream (NULL: the context's). */
int fk_stream_sync(fk_ctx *ctx, fk_stream *stream);

/* Launch. --------------------------------------------------------------------
 * `groups` threadgroups of `threads` threads, `lds_bytes` of dynamic
 * threadgroup memory, and the kernarg bytes: the buffers' device addresses
 * in binding order, then the parameter struct in C layout
 * (src/FuryKernel/Abi.hs:4-21,113-133).  A launch of zero groups does
 * nothing and returns FK_OK (src/FuryKernel/Backend.hs:84-87).  More than
 * 1024 threads or 160 KiB of threadgroup memory is FK_ERR_RANGE. */
int fk_launch(fk_fn *fn, uint32_t groups, uint32_t threads, uint32_t lds_bytes, const void *kernarg,
              size_t kernarg_bytes, fk_stream *stream);

/* The manifest: what each kernel of the code objects is. --------------------
 * A kernel's ABI is its buffers in binding order (name, access, type,
 * alignment), then its parameter struct's fields at their C offsets
 * (fkrocm_kernels.h) and the struct's size; its hash is 64-bit FNV-1a over
 * the canonical text `fk_abi_description` writes (src/FuryKernel/Abi.hs:
 * 98-133,135-162,255-262), so a `LoweredKernel`'s `lkAbi` hash and this
 * library's agree exactly when both describe one interface. */

typedef struct fk_abi_buffer {
  const char *name;
  const char *access; /* "read", "write", "read_write" */
  const char *type;   /* "f32", "f16", "bf16", "i8", "u32", "u64", ... */
  uint32_t align;     /* bytes */
} fk_abi_buffer;

typedef struct fk_abi_param {
  const char *name;
  const char *type;
  uint32_t offset; /* bytes into the struct */
} fk_abi_param;

typedef struct fk_kernel_abi {
  const char *entry;
  uint32_t threads; /* the threads every launch has; 0: any count up to 1024 */
  uint32_t n_buffers;
  const fk_abi_buffer *buffers;
  uint32_t n_params;
  const fk_abi_param *params;
  uint32_t params_size;
  uint64_t abi_hash;
} fk_kernel_abi;

/* 64-bit FNV-1a (src/FuryKernel/Abi.hs:255-262). */
uint64_t fk_fnv1a64(const void *bytes, size_t n);
/* The canonical text of an ABI ("abi 1", its buffers, its params, "params
 * size"), written NUL-terminated into `out` (up to cap - 1 bytes); returns
 * its full length. */
size_t fk_abi_description(const fk_kernel_abi *abi, char *out, size_t cap);
uint64_t fk_abi_hash(const fk_kernel_abi *abi);
/* Every kernel of this library's code objects. */
int fk_manifest_count(void);
const fk_kernel_abi *fk_manifest_at(int index);
const fk_kernel_abi *fk_manifest_find(const char *entry);

/* A buffer a launch binds: its device address and the bytes it holds there. */
typedef struct fk_binding {
  uint64_t addr;
  uint64_t bytes;
} fk_binding;

/* The checks a launch table makes before it builds a launch (host only, no
 * GPU): `abi_hash` is the kernel's; the buffers and parameter bytes are its
 * count and size; the threads are what it is built for; every buffer its
 * kernel dereferences for this entry and these parameters is bound (a GEMV
 * step entry's `_p<pro>_e<epi>` modes must agree with its parameters, and
 * decide what it reads), 16-byte aligned, and, for the GEMV steps, the decode
 * attention, its combine and the token, holds every byte the kernel touches.
 * FK_OK, or a status with the reason in `err`. */
int fk_launch_check(const char *entry, uint32_t groups, uint32_t threads, uint32_t lds_bytes,
                    const fk_binding *buffers, uint32_t n_buffers, const void *params, size_t params_bytes,
                    uint64_t abi_hash, char *err, size_t err_cap);

/* Launch tables: a planned step's launches, each checked once and kept with
 * its kernarg, queued in order by one call (the per-token path of a
 * `Backend`'s `loweredKernels`, src/FuryKernel/Backend.hs:76-101). --------- */

typedef struct fk_table fk_table;

int fk_table_create(fk_ctx *ctx, fk_table **out);
int fk_table_destroy(fk_table *table);
/* Appends a launch of `fn` after `fk_launch_check` passes; its index into
 * `*index` (may be NULL).  Zero groups: kept, and skipped when queued. */
int fk_table_add(fk_table *table, fk_fn *fn, uint32_t groups, uint32_t threads, uint32_t lds_bytes,
                 const fk_binding *buffers, uint32_t n_buffers, const void *params, size_t params_bytes,
                 uint64_t abi_hash, uint32_t *index);
int fk_table_count(const fk_table *table, uint32_t *count);
/* Queues launches [first, first + count) in order on the stream (a graph
 * capture records them). */
int fk_table_enqueue(fk_table *table, uint32_t first, uint32_t count, fk_stream *stream);

/* Events, for timing on the stream the kernels run on. */
int fk_event_create(fk_ctx *ctx, fk_event **out);
int fk_event_destroy(fk_event *event);
int fk_event_record(fk_event *event, fk_stream *stream);
int fk_event_sync(fk_event *event);
/* Work queued on `stream` after this call waits for the event's last record
 * (cross-stream ordering; under graph capture, an edge of the graph). */
int fk_stream_wait_event(fk_stream *stream, fk_event *event);
/* Milliseconds from `start` to `end`, both recorded and complete. */
int fk_event_elapsed_ms(fk_event *start, fk_event *end, float *ms);

/* Graphs: a stream's launches and copies captured once (a planned step's
 * launch list) and replayed, with the buffers they were captured with. */
int fk_graph_begin(fk_ctx *ctx, fk_stream *stream);
int fk_graph_end(fk_ctx *ctx, fk_stream *stream, fk_graph **out);
int fk_graph_replay(fk_graph *graph, fk_stream *stream);
int fk_graph_destroy(fk_graph *graph);

#ifdef __cplusplus
}
#endif

#endif /* FKROCM_H */
