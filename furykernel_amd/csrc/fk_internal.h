// fk_internal.h — the runtime's handle types, shared by the C ABI's
// translation units (fk_runtime.cpp, fk_ops.hip); not part of the ABI.
#pragma once

#include <hip/hip_runtime_api.h>

#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/fkrocm.h"

struct fk_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string last_error;
  std::mutex mu;  // guards the ownership sets below
  std::set<fk_module *> modules;
  std::set<fk_buf *> buffers;
  std::set<fk_arena *> arenas;
  std::set<fk_stream *> streams;
  std::set<fk_event *> events;
  std::set<fk_graph *> graphs;
  std::set<fk_table *> tables;
  std::set<void *> host;
  // fk_attend_decode's workspace (grown on demand), and the address of the
  // no-alloc entry's static scratch on this context's device.
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
  std::mutex workspace_mu;  // held across a call's grow and launch, so no thread frees it under another's launch
  void *scratch = nullptr;
};

struct fk_module {
  fk_ctx *ctx;
  hipModule_t mod;
  std::vector<fk_fn *> fns;
};

struct fk_fn {
  fk_module *mod;
  hipFunction_t fn;
  std::string entry;
};

struct fk_buf {
  fk_ctx *ctx;
  fk_arena *arena;  // null when the buffer owns its memory
  void *ptr;
  size_t size;
};

struct fk_arena {
  fk_ctx *ctx;
  void *base;
  size_t capacity;
  size_t used;
  std::vector<fk_buf *> handed;
};

struct fk_stream {
  fk_ctx *ctx;
  hipStream_t stream;
};

struct fk_event {
  fk_ctx *ctx;
  hipEvent_t event;
};

struct fk_graph {
  fk_ctx *ctx;
  hipGraph_t graph;
  hipGraphExec_t exec;
};

struct fk_table {
  struct Launch {
    fk_fn *fn;
    uint32_t groups, threads, lds_bytes;
    std::vector<unsigned char> kernarg;
  };
  fk_ctx *ctx;
  std::vector<Launch> launches;
};


// A failure's status and message, kept on the context (fk_runtime.cpp).
int fk_fail(fk_ctx *ctx, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
// The context's set-up and tear-down of the operations' memory (fk_ops.hip):
// the static scratch's address on the context's device, and the workspace.
int fk_ops_setup(fk_ctx *ctx);
void fk_ops_teardown(fk_ctx *ctx);
