// fk_manifest.cpp — what each kernel of the target's code objects is: its
// ABI (buffers in binding order with their access, type and alignment, then
// the parameter struct's fields at their C offsets), the canonical text the
// ABI hash covers and the hash itself (src/FuryKernel/Abi.hs:98-133,
// abiDescription :135-162, fnv1a64 :255-262), and the checks a launch table
// makes before it builds a launch's kernarg: the ABI hash the caller's
// lowering carries must be the kernel's, the buffers and parameter bytes must
// be the kernel's count and size, every buffer the kernel dereferences for its
// entry and parameters must be bound, and (for the GEMV step and the decode
// attention) every bound buffer must hold the bytes the kernel touches.
//
// Host code only: the checks run without a GPU.

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <deque>
#include <string>
#include <utility>
#include <vector>

#include "../../include/fkrocm.h"
#include "../../include/fkrocm_kernels.h"

namespace {

struct Entry {
  std::string entry;
  uint32_t threads = 0;
  std::vector<fk_abi_buffer> buffers;
  std::vector<fk_abi_param> params;
  uint32_t params_size = 0;
  fk_kernel_abi abi{};
};

// Strings the manifest points at live as long as it does (a deque never
// moves its elements).
const char *keep(const std::string &s) {
  static std::deque<std::string> kept;
  kept.push_back(s);
  return kept.back().c_str();
}

#define FK_P(S, f, ty) fk_abi_param{#f, ty, (uint32_t)offsetof(S, f)}
#define FK_PA(S, f, i, ty) fk_abi_param{#f "_" #i, ty, (uint32_t)(offsetof(S, f) + (i) * 4)}
#define FK_PX(S, f, name, ty) fk_abi_param{name, ty, (uint32_t)offsetof(S, f)}

fk_abi_buffer buf(const char *name, const char *access, const char *type) {
  return fk_abi_buffer{name, access, type, 16};
}

std::vector<fk_abi_param> attend_params() {
  using S = fk_step_attend_params;
  return {FK_P(S, heads, "u32"),    FK_P(S, kv_heads, "u32"), FK_P(S, head_dim, "u32"), FK_P(S, length, "u32"),
          FK_P(S, slots, "u32"),    FK_P(S, splits, "u32"),   FK_P(S, split, "u32"),    FK_P(S, rope, "u32"),
          FK_P(S, rotated, "u32"),  FK_P(S, rope_rows, "u32"), FK_P(S, scale, "f32"),   FK_P(S, window, "u32"),
          FK_P(S, cache_bf16, "u32"), FK_P(S, store, "u32"),  FK_P(S, krope, "u32"),    FK_P(S, has_reach, "u32")};
}

std::vector<fk_abi_param> store_params() {
  using S = fk_step_store_params;
  return {FK_P(S, n_stores, "u32"), FK_PA(S, rope, 0, "u32"), FK_PA(S, rope, 1, "u32"), FK_P(S, kv_heads, "u32"),
          FK_P(S, head_dim, "u32"), FK_P(S, length, "u32"),   FK_P(S, slots, "u32"),    FK_P(S, rotated, "u32"),
          FK_P(S, rope_rows, "u32"), FK_P(S, cache_bf16, "u32")};
}

// The paging fields of a params struct S that ends in an fk_paging g.
template <typename S>
std::vector<fk_abi_param> with_paging(std::vector<fk_abi_param> v) {
  v.push_back(FK_PX(S, g.block_size, "block_size", "u32"));
  v.push_back(FK_PX(S, g.table_len, "table_len", "u32"));
  v.push_back(FK_PX(S, g.blocks, "blocks", "u32"));
  return v;
}

std::vector<fk_abi_param> gemv_step_params() {
  using S = fk_step_gemv_params;
  return {FK_P(S, n_anchors, "u32"),   FK_PA(S, rows, 0, "u32"),      FK_PA(S, rows, 1, "u32"),
          FK_PA(S, rows, 2, "u32"),    FK_PA(S, first_row, 0, "u32"), FK_PA(S, first_row, 1, "u32"),
          FK_PA(S, first_row, 2, "u32"), FK_PA(S, first_row, 3, "u32"), FK_P(S, k, "u32"),
          FK_P(S, pro_mode, "u32"),    FK_P(S, seg, "u32"),           FK_P(S, eps, "f32"),
          FK_P(S, factor, "f32"),      FK_P(S, gfactor, "f32"),       FK_P(S, has_gamma, "u32"),
          FK_P(S, epi_mode, "u32"),    FK_P(S, store_tile, "u32"),    FK_P(S, table_rows, "u32"),
          FK_P(S, blocks, "u32"),      FK_P(S, arg_slots, "u32"),      FK_P(S, act, "u32"),
          FK_P(S, src2_off, "u32"),    FK_P(S, cap, "f32"),            FK_P(S, splits, "u32"),
          FK_P(S, head_dim, "u32")};
}

std::vector<fk_abi_param> gemm_params() {
  using S = fk_gemm_params;
  return {FK_P(S, m, "u32"),          FK_P(S, k, "u32"),          FK_P(S, n_anchors, "u32"),
          FK_PA(S, first_col, 0, "u32"), FK_PA(S, first_col, 1, "u32"), FK_PA(S, first_col, 2, "u32"),
          FK_PA(S, first_col, 3, "u32"), FK_PA(S, ldc, 0, "u32"),       FK_PA(S, ldc, 1, "u32"),
          FK_PA(S, ldc, 2, "u32"),     FK_P(S, act, "u32")};
}

std::vector<Entry> build() {
  std::vector<Entry> out;
  auto add = [&](const std::string &entry, uint32_t threads, std::vector<fk_abi_buffer> b,
                 std::vector<fk_abi_param> p, uint32_t size) {
    Entry e;
    e.entry = entry;
    e.threads = threads;
    e.buffers = std::move(b);
    e.params = std::move(p);
    e.params_size = size;
    out.push_back(std::move(e));
  };

  // The standalone GEMVs, RMSNorm, softmax and helpers.
  for (const char *wt : {"f32", "f16"})
    for (int r : {1, 2, 4})
      add(std::string("fk_gemv_") + wt + "_f32_r" + std::to_string(r), 0,
          {buf("w", "read", wt), buf("x", "read", "f32"), buf("y", "write", "f32")},
          {FK_P(fk_gemv_params, n, "u32"), FK_P(fk_gemv_params, k, "u32")}, sizeof(fk_gemv_params));
  for (const char *wt : {"f32", "f16", "bf16"})
    add(std::string("fk_gemv_p4_") + wt, 0, {buf("w", "read", wt), buf("x", "read", "f32"), buf("y", "write", "f32")},
        {FK_P(fk_gemv_params, n, "u32"), FK_P(fk_gemv_params, k, "u32")}, sizeof(fk_gemv_params));
  for (int r : {1, 2, 4})
    add("fk_gemv_i8_f16_r" + std::to_string(r), 0,
        {buf("w", "read", "i8"), buf("scale", "read", "f32"), buf("x", "read", "f16"), buf("y", "write", "f32")},
        {FK_P(fk_gemv_params, n, "u32"), FK_P(fk_gemv_params, k, "u32")}, sizeof(fk_gemv_params));
  {
    using S = fk_rmsnorm_params;
    add("fk_rmsnorm_f32", 0, {buf("x", "read", "f32"), buf("gamma", "read", "f32"), buf("y", "write", "f32")},
        {FK_P(S, rows, "u32"), FK_P(S, width, "u32"), FK_P(S, seg, "u32"), FK_P(S, eps, "f32"),
         FK_P(S, factor, "f32"), FK_P(S, has_gamma, "u32")},
        sizeof(S));
  }
  add("fk_softmax_f32", 0, {buf("x", "read", "f32"), buf("y", "write", "f32")},
      {FK_P(fk_softmax_params, rows, "u32"), FK_P(fk_softmax_params, n, "u32")}, sizeof(fk_softmax_params));
  add("fk_fill_u32", 0, {buf("dst", "write", "u32")},
      {FK_P(fk_fill_params, count, "u32"), FK_P(fk_fill_params, value, "u32")}, sizeof(fk_fill_params));
  add("fk_noop", 0, {}, {FK_P(fk_noop_params, unused, "u32")}, sizeof(fk_noop_params));
  add("fk_stream_read", 0, {buf("src", "read", "u32"), buf("out", "write", "u32")},
      {FK_P(fk_stream_read_params, words, "u64")}, sizeof(fk_stream_read_params));
  {
    using S = fk_init_normal_params;
    add("fk_init_normal", 0, {buf("dst", "write", "f32")},
        {FK_P(S, count, "u64"), FK_P(S, seed, "u64"), FK_P(S, std, "f32"), FK_P(S, dtype, "u32")}, sizeof(S));
  }

  // The GEMV step: every shape with every prologue and epilogue it is built for.
  struct Shape {
    const char *name, *wt;
    bool pairs;
  };
  const Shape shapes[] = {{"fk_step_gemv_f16_k2048_r1", "f16", true}, {"fk_step_gemv_f16_k2048_r2", "f16", true},
                          {"fk_step_gemv_f16_k8192_r1", "f16", false}, {"fk_step_gemv_bf16_k2048_r1", "bf16", true},
                          {"fk_step_gemv_bf16_k2048_r2", "bf16", true}, {"fk_step_gemv_bf16_k8192_r1", "bf16", false},
                          {"fk_step_gemv_f32_k256_r1", "f32", true},
                          {"fk_step_gemv_f32_k256_r2", "f32", true},   {"fk_step_gemv_f32_k1024_r1", "f32", true},
                          {"fk_step_gemv_f32_k1024_r2", "f32", true}};
  for (const Shape &s : shapes) {
    const char *wt = keep(s.wt);
    std::vector<fk_abi_buffer> b = {
        buf("w0", "read", wt),        buf("w1", "read", wt),         buf("w2", "read", wt),
        buf("y0", "write", "f32"),    buf("y1", "write", "f32"),     buf("y2", "write", "f32"),
        buf("src", "read", "f32"),    buf("src2", "read", "f32"),    buf("gamma", "read", "f32"),
        buf("table", "read", wt),     buf("token", "read", "u32"),   buf("res", "read", "f32"),
        buf("res_table", "read", wt), buf("res_token", "read", "u32"), buf("epi_out", "write", "f32"),
        buf("arg", "read_write", "u64")};
    for (int pro = 0; pro < 6; pro++)
      for (int epi = 0; epi < 6; epi++) {
        if (epi == FK_EPI_SILU_MUL && !s.pairs) continue;
        add(std::string(s.name) + "_p" + std::to_string(pro) + "_e" + std::to_string(epi), 512, b,
            gemv_step_params(), sizeof(fk_step_gemv_params));
      }
  }
  {
    using S = fk_step_token_params;
    add("fk_step_token", 64,
        {buf("arg", "read", "u64"), buf("out", "write", "u32"), buf("token", "write", "u32"),
         buf("position", "read_write", "u32")},
        {FK_P(S, slots, "u32"), FK_P(S, context, "u32"), FK_P(S, step, "u32"), FK_P(S, advance, "u32")}, sizeof(S));
  }
  {
    using S = fk_step_store_params;
    add("fk_step_store", 0,
        {buf("x0", "read", "f32"), buf("x1", "read", "f32"), buf("c0", "read_write", "f16"),
         buf("c1", "read_write", "f16"), buf("position", "read", "u32"), buf("slot", "read", "u32"),
         buf("rope", "read", "f32")},
        store_params(), sizeof(S));
  }
  add("fk_step_store_paged", 0,
      {buf("x0", "read", "f32"), buf("x1", "read", "f32"), buf("p0", "read", "u64"), buf("p1", "read", "u64"),
       buf("position", "read", "u32"), buf("table", "read", "u32"), buf("rope", "read", "f32")},
      with_paging<fk_step_store_paged_params>(store_params()), sizeof(fk_step_store_paged_params));
  {
    using S = fk_step_attend_params;
    add("fk_step_attend", 0,
        {buf("q", "read", "f32"), buf("knew", "read", "f32"), buf("vnew", "read", "f32"),
         buf("kc", "read_write", "f16"), buf("vc", "read_write", "f16"), buf("position", "read", "u32"),
         buf("slot", "read", "u32"), buf("rope", "read", "f32"), buf("partials", "write", "f32"),
         buf("reach", "read", "u32")},
        attend_params(), sizeof(S));
  }
  {
    using S = fk_step_attend_params;
    add("fk_step_attend_wide", 0,
        {buf("q", "read", "f32"), buf("knew", "read", "f32"), buf("vnew", "read", "f32"),
         buf("kc", "read_write", "f16"), buf("vc", "read_write", "f16"), buf("position", "read", "u32"),
         buf("slot", "read", "u32"), buf("rope", "read", "f32"), buf("partials", "write", "f32"),
         buf("reach", "read", "u32")},
        attend_params(), sizeof(S));
  }
  add("fk_step_attend_paged", 0,
      {buf("q", "read", "f32"), buf("knew", "read", "f32"), buf("vnew", "read", "f32"), buf("kpool", "read", "u64"),
       buf("vpool", "read", "u64"), buf("position", "read", "u32"), buf("table", "read", "u32"),
       buf("rope", "read", "f32"), buf("partials", "write", "f32"), buf("reach", "read", "u32")},
      with_paging<fk_step_attend_paged_params>(attend_params()), sizeof(fk_step_attend_paged_params));
  {
    using S = fk_step_combine_params;
    add("fk_step_combine", 64, {buf("partials", "read", "f32"), buf("out", "write", "f32")},
        {FK_P(S, heads, "u32"), FK_P(S, head_dim, "u32"), FK_P(S, splits, "u32")}, sizeof(S));
  }
  add("fk_step_argmax", 0, {buf("x", "read", "f32"), buf("out", "write", "u32")},
      {FK_P(fk_step_argmax_params, n, "u32")}, sizeof(fk_step_argmax_params));
  add("fk_step_act_mul", 0, {buf("a", "read", "f32"), buf("b", "read", "f32"), buf("y", "write", "f32")},
      {FK_P(fk_step_act_mul_params, n, "u32"), FK_P(fk_step_act_mul_params, act, "u32"),
       FK_P(fk_step_act_mul_params, b_off, "u32"), FK_P(fk_step_act_mul_params, half, "u32")},
      sizeof(fk_step_act_mul_params));
  add("fk_step_route", 64,
      {buf("x", "read", "f32"), buf("scale", "read", "f32"), buf("ids", "write", "u32"), buf("ws", "write", "f32")},
      {FK_P(fk_step_route_params, n, "u32"), FK_P(fk_step_route_params, k, "u32"),
       FK_P(fk_step_route_params, has_scale, "u32")},
      sizeof(fk_step_route_params));
  add("fk_step_combine_ranks", 0,
      {buf("w", "read", "f32"), buf("x", "read", "f32"), buf("res", "read", "f32"), buf("y", "write", "f32")},
      {FK_P(fk_step_combine_ranks_params, seg, "u32"), FK_P(fk_step_combine_ranks_params, ranks, "u32"),
       FK_P(fk_step_combine_ranks_params, residual, "u32")},
      sizeof(fk_step_combine_ranks_params));
  add("fk_step_elementwise", 0,
      {buf("a", "read", "f32"), buf("b", "read", "f32"), buf("c", "read", "f32"), buf("y", "write", "f32")},
      {FK_P(fk_step_elementwise_params, n, "u32"), FK_P(fk_step_elementwise_params, op, "u32"),
       FK_P(fk_step_elementwise_params, width, "u32"), FK_P(fk_step_elementwise_params, width_b, "u32"),
       FK_P(fk_step_elementwise_params, factor, "f32")},
      sizeof(fk_step_elementwise_params));
  for (const auto &g : {std::pair<const char *, const char *>{"fk_step_gather_f32", "f32"},
                        {"fk_step_gather_f16", "f16"}, {"fk_step_gather_bf16", "bf16"}}) {
    using S = fk_step_gather_params;
    add(g.first, 0, {buf("table", "read", g.second), buf("tokens", "read", "u32"), buf("y", "write", "f32")},
        {FK_P(S, rows, "u32"), FK_P(S, width, "u32"), FK_P(S, count, "u32"), FK_P(S, table_rows, "u32"),
         FK_P(S, factor, "f32")},
        sizeof(S));
  }
  for (const char *name : {"fk_gemv_routed_f16_r1", "fk_gemv_routed_f16_r2", "fk_gemv_routed_f32_r1",
                           "fk_gemv_routed_bf16_r1", "fk_gemv_routed_bf16_r2"}) {
    using S = fk_gemv_routed_params;
    add(name, 0,
        {buf("table", "read", "u64"), buf("ids", "read", "u32"), buf("x", "read", "f32"), buf("y", "write", "f32")},
        {FK_P(S, n, "u32"), FK_P(S, k, "u32"), FK_P(S, ranks, "u32"), FK_P(S, shared, "u32"), FK_P(S, entries, "u32"),
         FK_P(S, groups_per_rank, "u32")},
        sizeof(S));
  }
  add("fk_step_advance", 0,
      {buf("next_token", "read", "u32"), buf("token", "write", "u32"), buf("position", "read_write", "u32")},
      {FK_P(fk_step_advance_params, context, "u32"), FK_P(fk_step_advance_params, step, "u32")},
      sizeof(fk_step_advance_params));

  // The prefill.
  for (const char *mode : {"store", "add", "silu_mul"}) {
    const char *ct = std::strcmp(mode, "silu_mul") == 0 ? "f16" : "f32";
    add(std::string("fk_gemm_f16_") + mode, 256,
        {buf("a", "read", "f16"), buf("b0", "read", "f16"), buf("b1", "read", "f16"), buf("b2", "read", "f16"),
         buf("c0", "write", ct), buf("c1", "write", ct), buf("c2", "write", ct), buf("r0", "read", "f32")},
        gemm_params(), sizeof(fk_gemm_params));
  }
  add("fk_gemm_f16_store_keys", 256,
      {buf("a", "read", "f16"), buf("b0", "read", "f16"), buf("b1", "read", "f16"), buf("b2", "read", "f16"),
       buf("c0", "write", "f32"), buf("c1", "write", "f32"), buf("c2", "write", "f32"), buf("r0", "read", "f32"),
       buf("keys", "write", "u64")},
      gemm_params(), sizeof(fk_gemm_params));
  {
    using S = fk_gemm_qkv_params;
    std::vector<fk_abi_param> p = gemm_params();
    p.push_back(fk_abi_param{"kv_heads", "u32", (uint32_t)(offsetof(S, r) + offsetof(fk_gemm_rope_params, kv_heads))});
    p.push_back(fk_abi_param{"rope_rows", "u32", (uint32_t)(offsetof(S, r) + offsetof(fk_gemm_rope_params, rope_rows))});
    p.push_back(fk_abi_param{"length", "u32", (uint32_t)(offsetof(S, r) + offsetof(fk_gemm_rope_params, length))});
    p.push_back(fk_abi_param{"slots", "u32", (uint32_t)(offsetof(S, r) + offsetof(fk_gemm_rope_params, slots))});
    p.push_back(fk_abi_param{"cache_bf16", "u32", (uint32_t)(offsetof(S, r) + offsetof(fk_gemm_rope_params, cache_bf16))});
    p.push_back(fk_abi_param{"staged", "u32", (uint32_t)(offsetof(S, r) + offsetof(fk_gemm_rope_params, staged))});
    add("fk_gemm_f16_qkv_rope", 256,
        {buf("a", "read", "f16"), buf("b0", "read", "f16"), buf("b1", "read", "f16"), buf("b2", "read", "f16"),
         buf("c0", "write", "f16"), buf("c1", "read_write", "f16"), buf("c2", "read_write", "f16"),
         buf("r0", "read", "f32"), buf("position", "read", "u32"), buf("slot", "read", "u32"),
         buf("rope", "read", "f32")},
        p, sizeof(S));
    using SP = fk_gemm_qkv_paged_params;
    p.push_back(fk_abi_param{"block_size", "u32", (uint32_t)(offsetof(SP, pg) + offsetof(fk_paging, block_size))});
    p.push_back(fk_abi_param{"table_len", "u32", (uint32_t)(offsetof(SP, pg) + offsetof(fk_paging, table_len))});
    p.push_back(fk_abi_param{"blocks", "u32", (uint32_t)(offsetof(SP, pg) + offsetof(fk_paging, blocks))});
    add("fk_gemm_f16_qkv_rope_paged", 256,
        {buf("a", "read", "f16"), buf("b0", "read", "f16"), buf("b1", "read", "f16"), buf("b2", "read", "f16"),
         buf("c0", "write", "f16"), buf("c1", "read_write", "f16"), buf("c2", "read_write", "f16"),
         buf("r0", "read", "f32"), buf("position", "read", "u32"), buf("table", "read", "u32"),
         buf("rope", "read", "f32")},
        p, sizeof(SP));
  }
  {
    using S = fk_prefill_gather_params;
    add("fk_prefill_gather", 256, {buf("table", "read", "f16"), buf("tokens", "read", "u32"), buf("x", "write", "f32")},
        {FK_P(S, rows, "u32"), FK_P(S, width, "u32"), FK_P(S, table_rows, "u32"), FK_P(S, table_f16, "u32"),
         FK_P(S, factor, "f32")},
        sizeof(S));
  }
  {
    using S = fk_prefill_norm_params;
    const std::vector<fk_abi_param> p = {FK_P(S, rows, "u32"), FK_P(S, width, "u32"), FK_P(S, eps, "f32"),
                                         FK_P(S, factor, "f32"), FK_P(S, has_gamma, "u32")};
    const std::vector<fk_abi_buffer> b = {buf("x", "read", "f32"), buf("gamma", "read", "f32"), buf("y", "write", "f16")};
    add("fk_prefill_norm_pack", 256, b, p, sizeof(S));
    for (int w : {512, 1024, 2048, 4096}) add("fk_prefill_norm_pack_w" + std::to_string(w), 256, b, p, sizeof(S));
  }
  {
    using S = fk_prefill_rope_params;
    add("fk_prefill_rope_store", 0,
        {buf("q", "read", "f32"), buf("k", "read", "f32"), buf("v", "read", "f32"), buf("position", "read", "u32"),
         buf("slot", "read", "u32"), buf("rope", "read", "f32"), buf("qr", "write", "f16"),
         buf("kc", "read_write", "f16"), buf("vc", "read_write", "f16")},
        {FK_P(S, rows, "u32"), FK_P(S, heads, "u32"), FK_P(S, kv_heads, "u32"), FK_P(S, head_dim, "u32"),
         FK_P(S, rotated, "u32"), FK_P(S, rope_rows, "u32"), FK_P(S, length, "u32"), FK_P(S, slots, "u32"),
         FK_P(S, cache_bf16, "u32"), FK_P(S, staged, "u32")},
        sizeof(S));
  }
  {
    using S = fk_prefill_rope_paged_params;
    add("fk_prefill_rope_store_paged", 0,
        {buf("q", "read", "f32"), buf("k", "read", "f32"), buf("v", "read", "f32"), buf("position", "read", "u32"),
         buf("table", "read", "u32"), buf("rope", "read", "f32"), buf("qr", "write", "f16"),
         buf("kc", "read_write", "f16"), buf("vc", "read_write", "f16")},
        {FK_P(S, r.rows, "u32"), FK_P(S, r.heads, "u32"), FK_P(S, r.kv_heads, "u32"), FK_P(S, r.head_dim, "u32"),
         FK_P(S, r.rotated, "u32"), FK_P(S, r.rope_rows, "u32"), FK_P(S, r.length, "u32"), FK_P(S, r.slots, "u32"),
         FK_P(S, r.cache_bf16, "u32"), FK_P(S, r.staged, "u32"), FK_P(S, g.block_size, "u32"),
         FK_P(S, g.table_len, "u32"), FK_P(S, g.blocks, "u32")},
        sizeof(S));
  }
  {
    using S = fk_prefill_land_params;
    add("fk_prefill_land", 256,
        {buf("ks", "read", "f16"), buf("vs", "read", "f16"), buf("position", "read", "u32"),
         buf("slot", "read", "u32"), buf("kc", "read_write", "f16"), buf("vc", "read_write", "f16")},
        {FK_P(S, rows, "u32"), FK_P(S, kv_heads, "u32"), FK_P(S, head_dim, "u32"), FK_P(S, length, "u32"),
         FK_P(S, slots, "u32")},
        sizeof(S));
  }
  {
    using S = fk_prefill_attend_params;
    for (const char *form : {"fk_prefill_attend_g", "fk_prefill_attend_f16_g"})
    for (int g : {1, 2, 4})
      add(form + std::to_string(g), 64 * g,
          {buf("qr", "read", "f16"), buf("kc", "read", "f16"), buf("vc", "read", "f16"),
           buf("position", "read", "u32"), buf("slot", "read", "u32"), buf("out", "write", "f16"),
           buf("ks", "read", "f16"), buf("vs", "read", "f16")},
          {FK_P(S, rows, "u32"), FK_P(S, heads, "u32"), FK_P(S, kv_heads, "u32"), FK_P(S, length, "u32"),
           FK_P(S, slots, "u32"), FK_P(S, window, "u32"), FK_P(S, cache_bf16, "u32"), FK_P(S, scale, "f32"),
           FK_P(S, staged, "u32"), FK_P(S, run_rows, "u32")},
          sizeof(S));
  }
  {
    using S = fk_prefill_attend_paged_params;
    for (const char *form : {"fk_prefill_attend_paged_g", "fk_prefill_attend_paged_f16_g"})
    for (int g : {1, 2, 4})
      add(form + std::to_string(g), 64 * g,
          {buf("qr", "read", "f16"), buf("kc", "read", "f16"), buf("vc", "read", "f16"),
           buf("position", "read", "u32"), buf("table", "read", "u32"), buf("out", "write", "f16")},
          {FK_P(S, a.rows, "u32"), FK_P(S, a.heads, "u32"), FK_P(S, a.kv_heads, "u32"), FK_P(S, a.length, "u32"),
           FK_P(S, a.slots, "u32"), FK_P(S, a.window, "u32"), FK_P(S, a.cache_bf16, "u32"), FK_P(S, a.scale, "f32"),
           FK_P(S, a.staged, "u32"), FK_P(S, a.run_rows, "u32"), FK_P(S, g.block_size, "u32"),
           FK_P(S, g.table_len, "u32"), FK_P(S, g.blocks, "u32")},
          sizeof(S));
  }
  add("fk_prefill_softcap", 256, {buf("x", "read", "f32"), buf("y", "write", "f32")},
      {FK_P(fk_prefill_softcap_params, count, "u32"), FK_P(fk_prefill_softcap_params, cap, "f32")},
      sizeof(fk_prefill_softcap_params));
  add("fk_prefill_argmax", 256, {buf("x", "read", "f32"), buf("out", "write", "u32")},
      {FK_P(fk_prefill_argmax_params, rows, "u32"), FK_P(fk_prefill_argmax_params, width, "u32")},
      sizeof(fk_prefill_argmax_params));
  add("fk_prefill_argmax_keys", 256, {buf("keys", "read", "u64"), buf("out", "write", "u32")},
      {FK_P(fk_prefill_argmax_keys_params, rows, "u32"), FK_P(fk_prefill_argmax_keys_params, parts, "u32")},
      sizeof(fk_prefill_argmax_keys_params));

  for (Entry &e : out) {
    e.abi.entry = e.entry.c_str();
    e.abi.threads = e.threads;
    e.abi.n_buffers = (uint32_t)e.buffers.size();
    e.abi.buffers = e.buffers.data();
    e.abi.n_params = (uint32_t)e.params.size();
    e.abi.params = e.params.data();
    e.abi.params_size = e.params_size;
    e.abi.abi_hash = fk_abi_hash(&e.abi);
  }
  return out;
}

const std::vector<Entry> &manifest() {
  static const std::vector<Entry> m = build();
  return m;
}

std::string describe(const fk_kernel_abi *a) {
  std::string t = "abi 1\n";
  for (uint32_t i = 0; i < a->n_buffers; i++) {
    const fk_abi_buffer &b = a->buffers[i];
    t += std::string("buffer ") + b.name + " " + b.access + " " + b.type + " align " + std::to_string(b.align) + "\n";
  }
  for (uint32_t i = 0; i < a->n_params; i++) {
    const fk_abi_param &p = a->params[i];
    t += std::string("param ") + p.name + " " + p.type + " at " + std::to_string(p.offset) + "\n";
  }
  t += "params size " + std::to_string(a->params_size) + "\n";
  return t;
}

// Launch checks ---------------------------------------------------------------

int bad(char *err, size_t cap, int code, const char *fmt, ...) __attribute__((format(printf, 4, 5)));
int bad(char *err, size_t cap, int code, const char *fmt, ...) {
  if (err && cap) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, cap, fmt, ap);
    va_end(ap);
  }
  return code;
}

int index_of(const fk_kernel_abi *a, const char *name) {
  for (uint32_t i = 0; i < a->n_buffers; i++)
    if (std::strcmp(a->buffers[i].name, name) == 0) return (int)i;
  return -1;
}

// The (prologue, epilogue) of a GEMV step entry: the suffix the kernel is
// specialised on.
bool gemv_modes(const char *entry, int *pro, int *epi, int *wbytes, int *kmax, int *r) {
  const char *pfx = "fk_step_gemv_";
  if (std::strncmp(entry, pfx, std::strlen(pfx)) != 0) return false;
  char wt[8] = {0};
  if (std::sscanf(entry + std::strlen(pfx), "%4[a-z0-9]_k%d_r%d_p%d_e%d", wt, kmax, r, pro, epi) != 5) return false;
  *wbytes = std::strcmp(wt, "f32") == 0 ? 4 : 2;
  return true;
}

struct Need {
  const char *name;
  uint64_t bytes;  // 0: only bound
};

}  // namespace

extern "C" {

uint64_t fk_fnv1a64(const void *bytes, size_t n) {
  const unsigned char *p = static_cast<const unsigned char *>(bytes);
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; i++) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

size_t fk_abi_description(const fk_kernel_abi *abi, char *out, size_t cap) {
  if (!abi) return 0;
  const std::string t = describe(abi);
  if (out && cap) {
    const size_t n = t.size() < cap - 1 ? t.size() : cap - 1;
    std::memcpy(out, t.data(), n);
    out[n] = '\0';
  }
  return t.size();
}

uint64_t fk_abi_hash(const fk_kernel_abi *abi) {
  if (!abi) return 0;
  const std::string t = describe(abi);
  return fk_fnv1a64(t.data(), t.size());
}

int fk_manifest_count(void) { return (int)manifest().size(); }

const fk_kernel_abi *fk_manifest_at(int i) {
  const auto &m = manifest();
  return i >= 0 && (size_t)i < m.size() ? &m[i].abi : nullptr;
}

const fk_kernel_abi *fk_manifest_find(const char *entry) {
  if (!entry) return nullptr;
  for (const Entry &e : manifest())
    if (e.entry == entry) return &e.abi;
  return nullptr;
}

int fk_launch_check(const char *entry, uint32_t groups, uint32_t threads, uint32_t lds_bytes,
                    const fk_binding *b, uint32_t n_buffers, const void *params, size_t params_bytes,
                    uint64_t abi_hash, char *err, size_t cap) {
  const fk_kernel_abi *a = fk_manifest_find(entry);
  if (!a) return bad(err, cap, FK_ERR_NOT_FOUND, "%s: no such kernel in the manifest", entry ? entry : "(null)");
  if (abi_hash != a->abi_hash)
    return bad(err, cap, FK_ERR_ARG, "%s: the launch's ABI hash 0x%016llx is not the kernel's 0x%016llx", entry,
               (unsigned long long)abi_hash, (unsigned long long)a->abi_hash);
  if (n_buffers != a->n_buffers)
    return bad(err, cap, FK_ERR_ARG, "%s: %u buffers bound, the kernel takes %u", entry, n_buffers, a->n_buffers);
  if (params_bytes != a->params_size || (a->params_size && !params))
    return bad(err, cap, FK_ERR_ARG, "%s: %zu parameter bytes, the kernel's struct is %u", entry, params_bytes,
               a->params_size);
  if (n_buffers && !b) return bad(err, cap, FK_ERR_ARG, "%s: null bindings", entry);
  if (threads == 0 || threads > 1024 || (a->threads && threads != a->threads))
    return bad(err, cap, FK_ERR_RANGE, "%s: %u threads a group (the kernel is built for %u)", entry, threads,
               a->threads);
  if (lds_bytes > 160 * 1024)
    return bad(err, cap, FK_ERR_RANGE, "%s: %u bytes of threadgroup memory, more than 160 KiB", entry, lds_bytes);
  (void)groups;

  std::vector<Need> need;
  int pro = 0, epi = 0, wb = 0, kmax = 0, r = 0;
  if (gemv_modes(entry, &pro, &epi, &wb, &kmax, &r)) {
    fk_step_gemv_params p;
    std::memcpy(&p, params, sizeof p);
    if ((int)p.pro_mode != pro || (int)p.epi_mode != epi)
      return bad(err, cap, FK_ERR_ARG, "%s runs prologue %d and epilogue %d; its parameters say %u and %u", entry,
                 pro, epi, p.pro_mode, p.epi_mode);
    if (p.n_anchors < 1 || p.n_anchors > 3 || p.k == 0 || (int)p.k > kmax)
      return bad(err, cap, FK_ERR_RANGE, "%s: %u anchors, k = %u (at most %d)", entry, p.n_anchors, p.k, kmax);
    uint64_t widest = 0;
    for (uint32_t j = 0; j < p.n_anchors; j++) widest = p.rows[j] > widest ? p.rows[j] : widest;
    // The SiLU·mul epilogue: two anchors of as many rows, in blocks of row
    // pairs (r 2) or of one row of each anchor in turn (r 1: blocks twice
    // the rows, so that a wavefront's partner is the next).
    if (epi == FK_EPI_SILU_MUL &&
        (p.n_anchors != 2 || p.rows[0] != p.rows[1] || (r == 1 && (uint64_t)p.blocks != 2ull * p.rows[0])))
      return bad(err, cap, FK_ERR_ARG, "%s: the SiLU·mul epilogue on %u anchors, %u blocks of %d", entry, p.n_anchors,
                 p.blocks, r);
    if (epi == FK_EPI_SOFTCAP && (p.n_anchors != 1 || !(p.cap > 0.0f && p.cap < __builtin_inff())))
      return bad(err, cap, FK_ERR_ARG, "%s: a softcap of %g on %u anchors", entry, (double)p.cap, p.n_anchors);
    if ((p.act != FK_ACT_SILU && p.act != FK_ACT_GELU_TANH) || p.src2_off % 4)
      return bad(err, cap, FK_ERR_ARG, "%s: activation %u, second row at %u", entry, p.act, p.src2_off);
    static const char *w[3] = {"w0", "w1", "w2"}, *y[3] = {"y0", "y1", "y2"};
    for (uint32_t j = 0; j < p.n_anchors; j++) {
      need.push_back({w[j], (uint64_t)p.rows[j] * p.k * wb});
      if (p.store_tile) need.push_back({y[j], (uint64_t)p.rows[j] * 4});
    }
    const uint64_t k4 = (uint64_t)p.k * 4;
    if (pro == FK_PRO_GATHER || pro == FK_PRO_GATHER_RMSNORM) {
      need.push_back({"table", (uint64_t)p.table_rows * p.k * wb});
      need.push_back({"token", 4});
    } else if (pro == FK_PRO_COMBINE) {
      if (p.splits < 1 || p.splits > 8 || p.head_dim == 0 || p.head_dim % 4 || p.k % p.head_dim)
        return bad(err, cap, FK_ERR_ARG, "%s: a combine of %u splits of heads of %u", entry, p.splits, p.head_dim);
      need.push_back({"src", (uint64_t)(p.k / p.head_dim) * p.splits * (p.head_dim + 2) * 4});
    } else {
      need.push_back({"src", k4});
    }
    if (pro == FK_PRO_SILU_MUL) need.push_back({"src2", k4 + (uint64_t)p.src2_off * 4});
    if (pro == FK_PRO_RMSNORM || pro == FK_PRO_GATHER_RMSNORM) need.push_back({"gamma", k4});
    if (epi == FK_EPI_ADD_STORED) {
      need.push_back({"res", widest * 4});
      need.push_back({"epi_out", widest * 4});
    } else if (epi == FK_EPI_ADD_GATHER) {
      need.push_back({"res_table", (uint64_t)p.table_rows * widest * wb});
      need.push_back({"res_token", 4});
      need.push_back({"epi_out", widest * 4});
    } else if (epi == FK_EPI_SILU_MUL) {
      need.push_back({"epi_out", (uint64_t)p.rows[0] * 4});
    } else if (epi == FK_EPI_ARGMAX) {
      need.push_back({"arg", (uint64_t)p.arg_slots * 8});
    } else if (epi == FK_EPI_SOFTCAP) {
      need.push_back({"epi_out", (uint64_t)p.rows[0] * 4});
      if (p.arg_slots) need.push_back({"arg", (uint64_t)p.arg_slots * 8});
    }
  } else if (std::strcmp(entry, "fk_step_attend") == 0 || std::strcmp(entry, "fk_step_attend_wide") == 0 ||
             std::strcmp(entry, "fk_step_attend_paged") == 0) {
    fk_step_attend_paged_params pp{};
    std::memcpy(&pp, params, std::strcmp(entry, "fk_step_attend_paged") == 0 ? sizeof pp : sizeof pp.a);
    const fk_step_attend_params &p = pp.a;
    const bool paged = entry[14] == '_' && entry[15] == 'p';
    const bool wide = entry[14] == '_' && entry[15] == 'w';
    // Wide splits: 64 positions a wavefront, up to 8 wavefronts, the LDS of
    // fk_attention.h's wide_lds_floats.
    const bool split_ok = wide ? (p.split % 64 == 0 && p.split == threads && threads >= 64 && threads <= 512 &&
                                  (p.head_dim == 16 || p.head_dim == 32 || p.head_dim == 64) &&
                                  (uint64_t)lds_bytes >= 4ull * (584 + (threads / 64) * (32 * 68 + 2 * 512 + 24)))
                               : (p.split == 64 || p.split == 128);
    if (p.kv_heads == 0 || p.heads % p.kv_heads || p.head_dim == 0 || p.head_dim > 64 || p.head_dim % 8 ||
        !split_ok || p.heads / p.kv_heads > 8 || groups != p.kv_heads * p.splits)
      return bad(err, cap, FK_ERR_ARG, "%s: %u heads over %u, width %u, splits of %u, %u groups for %u splits", entry,
                 p.heads, p.kv_heads, p.head_dim, p.split, groups, p.splits);
    if (paged) {
      if (pp.g.block_size == 0 || pp.g.table_len == 0 || pp.g.blocks == 0)
        return bad(err, cap, FK_ERR_ARG, "%s: blocks of %u positions, tables of %u of a pool of %u", entry,
                   pp.g.block_size, pp.g.table_len, pp.g.blocks);
      need = {{"q", (uint64_t)p.heads * p.head_dim * 4},
              {"kpool", (uint64_t)pp.g.blocks * 8},
              {"vpool", (uint64_t)pp.g.blocks * 8},
              {"position", 4},
              {"table", (uint64_t)pp.g.table_len * 4},
              {"partials", (uint64_t)p.heads * p.splits * (p.head_dim + 2) * 4}};
    } else {
      const uint64_t cache = (uint64_t)p.slots * p.kv_heads * p.length * p.head_dim * 2;
      need = {{"q", (uint64_t)p.heads * p.head_dim * 4},
              {"kc", cache},
              {"vc", cache},
              {"position", 4},
              {"slot", 4},
              {"partials", (uint64_t)p.heads * p.splits * (p.head_dim + 2) * 4}};
    }
    if (p.has_reach && wide)
      return bad(err, cap, FK_ERR_ARG, "%s: the wide splits take no reach", entry);
    if (p.has_reach) need.push_back({"reach", 4});
    if (p.store) {
      need.push_back({"knew", (uint64_t)p.kv_heads * p.head_dim * 4});
      need.push_back({"vnew", (uint64_t)p.kv_heads * p.head_dim * 4});
    }
    if (p.rope || p.krope) need.push_back({"rope", (uint64_t)p.rope_rows * p.rotated * 8});
  } else if (std::strcmp(entry, "fk_step_combine") == 0) {
    fk_step_combine_params p;
    std::memcpy(&p, params, sizeof p);
    // one wavefront a head
    if (p.heads == 0 || groups != p.heads || p.splits == 0 || p.head_dim == 0)
      return bad(err, cap, FK_ERR_ARG, "%s: %u heads of %u in %u splits, %u threadgroups", entry, p.heads,
                 p.head_dim, p.splits, groups);
    need = {{"partials", (uint64_t)p.heads * p.splits * (p.head_dim + 2) * 4},
            {"out", (uint64_t)p.heads * p.head_dim * 4}};
  } else if (std::strcmp(entry, "fk_step_store_paged") == 0) {
    fk_step_store_paged_params pp;
    std::memcpy(&pp, params, sizeof pp);
    if (pp.g.block_size == 0 || pp.g.table_len == 0 || pp.g.blocks == 0 || pp.s.n_stores < 1 || pp.s.n_stores > 2)
      return bad(err, cap, FK_ERR_ARG, "%s: %u stores, blocks of %u positions, tables of %u of a pool of %u", entry,
                 pp.s.n_stores, pp.g.block_size, pp.g.table_len, pp.g.blocks);
    const uint64_t row = (uint64_t)pp.s.kv_heads * pp.s.head_dim * 4;
    need = {{"x0", row}, {"p0", (uint64_t)pp.g.blocks * 8}, {"position", 4}, {"table", (uint64_t)pp.g.table_len * 4}};
    if (pp.s.n_stores > 1) {
      need.push_back({"x1", row});
      need.push_back({"p1", (uint64_t)pp.g.blocks * 8});
    }
    if (pp.s.rope[0] || pp.s.rope[1]) need.push_back({"rope", (uint64_t)pp.s.rope_rows * pp.s.rotated * 8});
  } else if (std::strcmp(entry, "fk_step_store") == 0) {
    fk_step_store_params p;
    std::memcpy(&p, params, sizeof p);
    need = {{"x0", 0}, {"c0", 0}, {"position", 4}, {"slot", 4}};
    if (p.n_stores > 1) {
      need.push_back({"x1", 0});
      need.push_back({"c1", 0});
    }
    if (p.rope[0] || p.rope[1]) need.push_back({"rope", 0});
  } else if (std::strcmp(entry, "fk_step_act_mul") == 0) {
    fk_step_act_mul_params p;
    std::memcpy(&p, params, sizeof p);
    if (p.n == 0 || (uint64_t)groups * threads < p.n || (p.half && p.n % p.half))
      return bad(err, cap, FK_ERR_ARG, "%s: %u elements in segments of %u, %u x %u threads", entry, p.n, p.half,
                 groups, threads);
    need = {{"a", (uint64_t)(p.half ? 2 : 1) * p.n * 4}, {"y", (uint64_t)p.n * 4}};
    if (!p.half) need.push_back({"b", ((uint64_t)p.b_off + p.n) * 4});
  } else if (std::strcmp(entry, "fk_step_route") == 0) {
    fk_step_route_params p;
    std::memcpy(&p, params, sizeof p);
    if (p.k < 1 || p.k > 8 || p.k > p.n)
      return bad(err, cap, FK_ERR_ARG, "%s: the %u largest of %u logits (1 to 8)", entry, p.k, p.n);
    need = {{"x", (uint64_t)p.n * 4}, {"ids", (uint64_t)p.k * 4}, {"ws", (uint64_t)p.k * 4}};
    if (p.has_scale) need.push_back({"scale", (uint64_t)p.n * 4});
  } else if (std::strcmp(entry, "fk_step_combine_ranks") == 0) {
    fk_step_combine_ranks_params p;
    std::memcpy(&p, params, sizeof p);
    if (p.ranks < 1 || p.seg == 0 || (uint64_t)groups * threads < p.seg)
      return bad(err, cap, FK_ERR_ARG, "%s: %u ranks of %u in %u x %u threads", entry, p.ranks, p.seg, groups,
                 threads);
    need = {{"w", (uint64_t)p.ranks * 4}, {"x", (uint64_t)p.ranks * p.seg * 4}, {"y", (uint64_t)p.seg * 4}};
    if (p.residual) need.push_back({"res", (uint64_t)p.seg * 4});
  } else if (std::strncmp(entry, "fk_gemv_p4_", 11) == 0) {
    fk_gemv_params p;
    std::memcpy(&p, params, sizeof p);
    const uint64_t eb = std::strcmp(entry + 11, "f32") == 0 ? 4 : 2;
    // a wavefront a row, packs of 4 elements
    if (p.n == 0 || p.k == 0 || p.k % 4 || threads % 64 || threads > 256 ||
        (uint64_t)groups * (threads / 64) < p.n)
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows of %u in %u groups of %u threads", entry, p.n, p.k, groups,
                 threads);
    need = {{"w", (uint64_t)p.n * p.k * eb}, {"x", (uint64_t)p.k * 4}, {"y", (uint64_t)p.n * 4}};
  } else if (std::strcmp(entry, "fk_step_elementwise") == 0) {
    fk_step_elementwise_params p;
    std::memcpy(&p, params, sizeof p);
    const uint64_t n = p.n;
    if (n == 0 || (uint64_t)groups * threads < n || p.op > FK_ELT_CONCAT || p.width == 0 ||
        (p.op == FK_ELT_STANDARDIZE && n % p.width) ||
        (p.op == FK_ELT_CONCAT && (p.width_b == 0 || n % (p.width + p.width_b))))
      return bad(err, cap, FK_ERR_ARG, "%s: operation %u over %u elements in rows of %u (+%u), %u x %u threads",
                 entry, p.op, p.n, p.width, p.width_b, groups, threads);
    need = {{"a", n * 4}, {"y", n * 4}};
    if (p.op == FK_ELT_ADD) need.push_back({"b", n * 4});
    if (p.op == FK_ELT_SCALE) need.push_back({"b", 4});
    if (p.op == FK_ELT_STANDARDIZE) {
      need.push_back({"b", (uint64_t)p.width * 4});
      need.push_back({"c", (uint64_t)p.width * 4});
    }
    if (p.op == FK_ELT_CONCAT) {
      const uint64_t rows = n / (p.width + p.width_b);
      need = {{"a", rows * p.width * 4}, {"b", rows * p.width_b * 4}, {"y", n * 4}};
    }
  } else if (std::strncmp(entry, "fk_step_gather_", 15) == 0) {
    fk_step_gather_params p;
    std::memcpy(&p, params, sizeof p);
    const uint64_t eb = std::strcmp(entry + 15, "f32") == 0 ? 4 : 2;
    const uint64_t n = (uint64_t)p.rows * p.width;
    if (n == 0 || p.count == 0 || p.table_rows == 0 || (uint64_t)groups * threads < n)
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows of %u, %u tokens a row of a table of %u, %u x %u threads", entry,
                 p.rows, p.width, p.count, p.table_rows, groups, threads);
    need = {{"table", (uint64_t)p.table_rows * p.width * eb}, {"tokens", (uint64_t)p.rows * p.count * 4},
            {"y", n * 4}};
  } else if (std::strncmp(entry, "fk_gemv_routed_", 15) == 0) {
    fk_gemv_routed_params p;
    std::memcpy(&p, params, sizeof p);
    const bool f32 = std::strncmp(entry + 15, "f32", 3) == 0;
    const uint32_t pack = f32 ? 4 : 8, r = (uint32_t)(entry[std::strlen(entry) - 1] - '0');
    if (p.entries == 0 || p.ranks == 0 || p.n == 0 || p.n % r || p.k == 0 || p.k % pack || threads % 64 ||
        threads > 256 ||
        p.groups_per_rank == 0 || groups != p.ranks * p.groups_per_rank ||
        (uint64_t)p.groups_per_rank * (threads / 64) * r < p.n)
      return bad(err, cap, FK_ERR_ARG, "%s: %u ranks of %u rows at k %u in %u groups of %u", entry, p.ranks, p.n,
                 p.k, groups, threads);
    need = {{"table", (uint64_t)p.entries * 8},
            {"ids", (uint64_t)p.ranks * 4},
            {"x", (uint64_t)(p.shared ? 1 : p.ranks) * p.k * 4},
            {"y", (uint64_t)p.ranks * p.n * 4}};
  } else if (std::strcmp(entry, "fk_step_token") == 0) {
    fk_step_token_params p;
    std::memcpy(&p, params, sizeof p);
    need = {{"arg", (uint64_t)p.slots * 8}, {"out", 4}};
    if (p.advance) {
      need.push_back({"token", 4});
      need.push_back({"position", 4});
    }
  } else if (std::strncmp(entry, "fk_gemm_f16_", 12) == 0) {
    fk_gemm_params p;
    std::memcpy(&p, params, sizeof p);
    static const char *bn[3] = {"b0", "b1", "b2"}, *cn[3] = {"c0", "c1", "c2"};
    // The tiles: 256 rows by 256 columns of the anchors (SiLU·mul: 128 gate
    // columns and their up columns), one threadgroup each, k in pairs of
    // steps of 32; the LDS ring of 4 stages.
    const bool silu = std::strcmp(entry, "fk_gemm_f16_silu_mul") == 0;
    const uint32_t cols = silu ? p.ldc[0] : (p.n_anchors >= 1 && p.n_anchors <= 3 ? p.first_col[p.n_anchors] : 0);
    const uint32_t unit = silu ? 128 : 256;
    bool shape = p.n_anchors >= 1 && p.n_anchors <= (silu ? 1u : 3u) && p.m && p.m % 256 == 0 && p.k &&
                 p.k % 64 == 0 && cols && cols % unit == 0 && (silu || p.first_col[0] == 0);
    for (uint32_t j = 0; shape && !silu && j < p.n_anchors; j++)
      shape = p.first_col[j + 1] > p.first_col[j] && (p.first_col[j + 1] - p.first_col[j]) % 256 == 0 &&
              p.ldc[j] >= p.first_col[j + 1] - p.first_col[j];
    if (!shape || (uint64_t)groups != (uint64_t)(p.m / 256) * (cols / unit))
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows, k %u, %u anchors over %u columns in %u threadgroups", entry, p.m,
                 p.k, p.n_anchors, cols, groups);
    const uint32_t lds = 4 * (256 + 256) * 32 * 2;
    if (lds_bytes < lds)
      return bad(err, cap, FK_ERR_RANGE, "%s: %u bytes of threadgroup memory, its ring takes %u", entry, lds_bytes,
                 lds);
    need.push_back({"a", 0});
    for (uint32_t j = 0; j < p.n_anchors && j < 3; j++) {
      need.push_back({bn[j], 0});
      need.push_back({cn[j], 0});
    }
    if (std::strcmp(entry, "fk_gemm_f16_add") == 0) need.push_back({"r0", 0});
    if (std::strcmp(entry, "fk_gemm_f16_store_keys") == 0) {
      // One anchor whose columns start at 0 and fill its rows: the keys
      // index a row's columns 128 at a time.
      if (p.n_anchors != 1 || p.first_col[0] != 0 || p.first_col[1] == 0 || p.ldc[0] != p.first_col[1] ||
          p.first_col[1] % 256 || p.m % 256)
        return bad(err, cap, FK_ERR_ARG, "%s: %u anchors, columns [%u, %u) in rows of %u", entry, p.n_anchors,
                   p.first_col[0], p.first_col[1], p.ldc[0]);
      need.push_back({"keys", (uint64_t)p.m * (p.ldc[0] / 128) * 8});
    }
    if (std::strcmp(entry, "fk_gemm_f16_qkv_rope") == 0) {
      need.push_back({"position", 0});
      need.push_back({"slot", 0});
      need.push_back({"rope", 0});
    }
    if (std::strcmp(entry, "fk_gemm_f16_qkv_rope_paged") == 0) {
      fk_gemm_qkv_paged_params q;
      std::memcpy(&q, params, sizeof q);
      if (q.pg.block_size == 0 || q.pg.table_len == 0 || q.pg.blocks == 0 || q.r.staged || q.r.kv_heads == 0)
        return bad(err, cap, FK_ERR_ARG, "%s: blocks of %u positions, tables of %u, a pool of %u, staged %u", entry,
                   q.pg.block_size, q.pg.table_len, q.pg.blocks, q.r.staged);
      const uint64_t pool = (uint64_t)q.pg.blocks * q.r.kv_heads * q.pg.block_size * 64 * 2;
      need.push_back({"position", (uint64_t)p.m * 4});
      need.push_back({"table", (uint64_t)p.m * q.pg.table_len * 4});
      need.push_back({"rope", 0});
      for (Need &n : need)
        if (std::strcmp(n.name, "c1") == 0 || std::strcmp(n.name, "c2") == 0) n.bytes = pool;
    }
  } else if (std::strncmp(entry, "fk_prefill_attend_g", 19) == 0 ||
             std::strncmp(entry, "fk_prefill_attend_f16_g", 23) == 0) {
    fk_prefill_attend_params p;
    std::memcpy(&p, params, sizeof p);
    // The f16 form loads f16 ring rows straight into LDS: no bf16 rows to
    // convert, no staged rows.
    if (entry[18] == 'f' && (p.cache_bf16 || p.staged))
      return bad(err, cap, FK_ERR_ARG, "%s: bf16 caches %u or staged rows %u", entry, p.cache_bf16, p.staged);
    const uint64_t kw = (uint64_t)p.kv_heads * 64 * 2;
    need = {{"qr", (uint64_t)p.rows * p.heads * 64 * 2},
            {"kc", (uint64_t)p.slots * p.length * kw},
            {"vc", (uint64_t)p.slots * p.length * kw},
            {"position", (uint64_t)p.rows * 4},
            {"slot", (uint64_t)p.rows * 4},
            {"out", (uint64_t)p.rows * p.heads * 64 * 2}};
    const uint32_t g = (uint32_t)(entry[std::strlen(entry) - 1] - '0');
    if ((p.staged && p.run_rows == 0) || (p.run_rows && (p.run_rows % 32 || p.rows % p.run_rows)) || p.rows % 32 ||
        p.rows == 0 || p.kv_heads == 0)
      return bad(err, cap, FK_ERR_ARG, "%s: runs of %u rows in a step of %u (multiples of 32 that divide it)", entry,
                 p.run_rows, p.rows);
    // The grid is every (query block, kv head), heaviest first: a larger
    // grid would index blocks past their run; the heads are the group's
    // wavefronts; keys go by blocks of 64 positions.
    if (p.heads != g * p.kv_heads || p.length == 0 || p.length % 64 || p.slots == 0 ||
        (uint64_t)groups != (uint64_t)(p.rows / 32) * p.kv_heads || threads != g * 64)
      return bad(err, cap, FK_ERR_ARG, "%s: %u heads over %u, a ring of %u, %u threadgroups of %u threads", entry,
                 p.heads, p.kv_heads, p.length, groups, threads);
    if (p.staged) {
      need.push_back({"ks", (uint64_t)p.rows * kw});
      need.push_back({"vs", (uint64_t)p.rows * kw});
    }
  } else if (std::strcmp(entry, "fk_prefill_argmax_keys") == 0) {
    fk_prefill_argmax_keys_params p;
    std::memcpy(&p, params, sizeof p);
    if (p.parts == 0 || (uint64_t)groups * 4 < p.rows || threads != 256)
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows of %u keys in %u x %u threads", entry, p.rows, p.parts, groups,
                 threads);
    need = {{"keys", (uint64_t)p.rows * p.parts * 8}, {"out", (uint64_t)p.rows * 4}};
  } else if (std::strcmp(entry, "fk_prefill_rope_store_paged") == 0) {
    fk_prefill_rope_paged_params pp;
    std::memcpy(&pp, params, sizeof pp);
    const fk_prefill_rope_params &p = pp.r;
    if (p.rows == 0 || groups != p.rows || p.staged || p.head_dim == 0 || p.kv_heads == 0 ||
        2 * p.rotated > p.head_dim || pp.g.block_size == 0 || pp.g.table_len == 0 || pp.g.blocks == 0)
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows in %u threadgroups, blocks of %u, tables of %u, staged %u", entry,
                 p.rows, groups, pp.g.block_size, pp.g.table_len, p.staged);
    const uint64_t kw = (uint64_t)p.kv_heads * p.head_dim;
    const uint64_t pool = (uint64_t)pp.g.blocks * p.kv_heads * pp.g.block_size * p.head_dim * 2;
    need = {{"q", (uint64_t)p.rows * p.heads * p.head_dim * 4}, {"k", (uint64_t)p.rows * kw * 4},
            {"v", (uint64_t)p.rows * kw * 4}, {"position", (uint64_t)p.rows * 4},
            {"table", (uint64_t)p.rows * pp.g.table_len * 4}, {"rope", (uint64_t)p.rope_rows * p.rotated * 8},
            {"qr", (uint64_t)p.rows * p.heads * p.head_dim * 2}, {"kc", pool}, {"vc", pool}};
  } else if (std::strncmp(entry, "fk_prefill_attend_paged_g", 25) == 0 ||
             std::strncmp(entry, "fk_prefill_attend_paged_f16_g", 29) == 0) {
    fk_prefill_attend_paged_params pp;
    std::memcpy(&pp, params, sizeof pp);
    const fk_prefill_attend_params &p = pp.a;
    const uint32_t g = (uint32_t)(entry[std::strlen(entry) - 1] - '0');
    // The f16 form loads f16 pool rows straight into LDS, at 32-bit offsets
    // into the pool, through a block table it holds in LDS (256 entries).
    if (entry[24] == 'f' &&
        (p.cache_bf16 || pp.g.table_len > 256 ||
         (uint64_t)pp.g.blocks * p.kv_heads * pp.g.block_size * 128 > 0xFFFFFFFFull))
      return bad(err, cap, FK_ERR_ARG, "%s: bf16 caches %u, tables of %u, a pool of %u blocks", entry, p.cache_bf16,
                 pp.g.table_len, pp.g.blocks);
    if (p.rows == 0 || p.rows % 32 || p.kv_heads == 0 || p.heads != g * p.kv_heads || p.staged ||
        (p.run_rows && (p.run_rows % 32 || p.rows % p.run_rows)) || pp.g.block_size == 0 || pp.g.table_len == 0 ||
        pp.g.blocks == 0 || groups != (p.rows / 32) * p.kv_heads)
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows, %u heads over %u, blocks of %u, tables of %u, %u threadgroups",
                 entry, p.rows, p.heads, p.kv_heads, pp.g.block_size, pp.g.table_len, groups);
    const uint64_t pool = (uint64_t)pp.g.blocks * p.kv_heads * pp.g.block_size * 64 * 2;
    need = {{"qr", (uint64_t)p.rows * p.heads * 64 * 2},
            {"kc", pool},
            {"vc", pool},
            {"position", (uint64_t)p.rows * 4},
            {"table", (uint64_t)p.rows * pp.g.table_len * 4},
            {"out", (uint64_t)p.rows * p.heads * 64 * 2}};
  } else if (std::strcmp(entry, "fk_prefill_rope_store") == 0) {
    fk_prefill_rope_params p;
    std::memcpy(&p, params, sizeof p);
    // One threadgroup a row.
    if (p.rows == 0 || groups != p.rows || p.head_dim == 0 || p.kv_heads == 0 || 2 * p.rotated > p.head_dim ||
        p.rope_rows == 0 || (!p.staged && (p.length == 0 || p.slots == 0)))
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows in %u threadgroups, heads of %u turning %u pairs, a ring of %u",
                 entry, p.rows, groups, p.head_dim, p.rotated, p.length);
    const uint64_t kw = (uint64_t)p.kv_heads * p.head_dim;
    const uint64_t cache = p.staged ? (uint64_t)p.rows * kw * 2 : (uint64_t)p.slots * p.length * kw * 2;
    need = {{"q", (uint64_t)p.rows * p.heads * p.head_dim * 4}, {"k", (uint64_t)p.rows * kw * 4},
            {"v", (uint64_t)p.rows * kw * 4}, {"position", (uint64_t)p.rows * 4},
            {"slot", (uint64_t)p.rows * 4}, {"rope", (uint64_t)p.rope_rows * p.rotated * 8},
            {"qr", (uint64_t)p.rows * p.heads * p.head_dim * 2}, {"kc", cache}, {"vc", cache}};
  } else if (std::strcmp(entry, "fk_prefill_land") == 0) {
    fk_prefill_land_params p;
    std::memcpy(&p, params, sizeof p);
    // One threadgroup a row.
    if (p.rows == 0 || groups != p.rows || p.kv_heads == 0 || p.head_dim == 0 || p.length == 0 || p.slots == 0)
      return bad(err, cap, FK_ERR_ARG, "%s: %u rows in %u threadgroups, %u heads of %u, a ring of %u in %u slots",
                 entry, p.rows, groups, p.kv_heads, p.head_dim, p.length, p.slots);
    const uint64_t kw = (uint64_t)p.kv_heads * p.head_dim * 2;
    need = {{"ks", (uint64_t)p.rows * kw}, {"vs", (uint64_t)p.rows * kw}, {"position", (uint64_t)p.rows * 4},
            {"slot", (uint64_t)p.rows * 4}, {"kc", (uint64_t)p.slots * p.length * kw},
            {"vc", (uint64_t)p.slots * p.length * kw}};
  } else {
    // Every other kernel dereferences each of its buffers (a norm without
    // gains excepted).
    bool gains = true;
    if (std::strcmp(entry, "fk_rmsnorm_f32") == 0) {
      fk_rmsnorm_params p;
      std::memcpy(&p, params, sizeof p);
      gains = p.has_gamma != 0;
    } else if (std::strncmp(entry, "fk_prefill_norm_pack", 20) == 0) {
      fk_prefill_norm_params p;
      std::memcpy(&p, params, sizeof p);
      gains = p.has_gamma != 0;
    }
    for (uint32_t i = 0; i < a->n_buffers; i++)
      if (gains || std::strcmp(a->buffers[i].name, "gamma") != 0) need.push_back({a->buffers[i].name, 0});
  }
  for (const Need &n : need) {
    const int i = index_of(a, n.name);
    if (i < 0) return bad(err, cap, FK_ERR_ARG, "%s: no buffer %s", entry, n.name);
    if (b[i].addr == 0)
      return bad(err, cap, FK_ERR_ARG, "%s: reads or writes %s, which the launch leaves unbound", entry, n.name);
    if (b[i].addr % a->buffers[i].align)
      return bad(err, cap, FK_ERR_ARG, "%s: %s at 0x%llx is not %u-byte aligned", entry, n.name,
                 (unsigned long long)b[i].addr, a->buffers[i].align);
    if (n.bytes && b[i].bytes < n.bytes)
      return bad(err, cap, FK_ERR_RANGE, "%s: %s holds %llu bytes, the kernel touches %llu", entry, n.name,
                 (unsigned long long)b[i].bytes, (unsigned long long)n.bytes);
  }
  return FK_OK;
}

}  // extern "C"
