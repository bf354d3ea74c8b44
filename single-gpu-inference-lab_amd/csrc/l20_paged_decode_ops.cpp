// TORCH_LIBRARY(l20_stack) binding of the MI355X paged decode ops.
//
// paged_decode_fp8_e4m3_split_out keeps the reference's schema verbatim
// (integrations/vllm/cuda/l20_paged_decode.cpp:128-135, relative to the
// reference repo root) and appends defaulted arguments, so every 13-argument
// legacy call still binds:
//   float? softmax_scale=None        (reference hard-codes 1/sqrt(128))
//   Tensor? k_scale_per_head=None    (fp32 [Hkv]; overrides k_scale)
//   Tensor? v_scale_per_head=None    (fp32 [Hkv]; overrides v_scale)
//   int q_len=1                      (query rows [B*q_len, Hq, D], causal)
//   Tensor(e!)? lse=None             (fp32 [B*q_len, Hq], natural log)
//   Tensor? tree_mask=None           (int32 [B, q_len] or [q_len] ancestor bitmasks over the
//                                     newest q_len keys: speculative tree verification)
// paged_decode_split_out (fp16/bf16 caches; schema :121-127) appends
// softmax_scale, q_len and lse the same way; paged_decode_split_indices_out
// is the CSR page-list variant the reference exports through pybind
// (l20_paged_decode.cpp:150-152, l20_paged_decode.cu:600-649), registered
// here with the same defaulted tail.
// The implementation validates with the reference's TORCH_CHECK messages
// (l20_paged_decode.cu:665-688) and calls the C ABI in
// libl20_paged_decode_hip.so on the current HIP stream.  Nothing is
// allocated: the caller owns the workspace, as in the reference.

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <optional>

#include "l20_kv_write.h"
#include "l20_paged_decode.h"
#include "l20_tree_verify.h"

namespace {

int32_t dtype_code(const at::Tensor &t) {
  switch (t.scalar_type()) {
    case at::kBFloat16:
      return L20_PD_BF16;
    case at::kHalf:
      return L20_PD_FP16;
    case at::kFloat:
      return L20_PD_FP32;
    default:
      return -1;
  }
}

void check_same_device(const at::Tensor &t, const at::Tensor &query, const char *what) {
  TORCH_CHECK(t.device() == query.device(), what, " must be on the query's device");
}

// Page addressing of one call: a [batch, max_pages] block table, or a CSR
// page list (page_indptr [batch + 1], page_indices flat).
struct PageTable {
  const at::Tensor *table;
  const at::Tensor *indptr;  // nullptr: block table
};

// Validation shared by the three ops and the argument block they pass to the
// C ABI.  Cache-dtype checks are done by the callers.
l20_pd_fp8_args make_args(const at::Tensor &query, const at::Tensor &key_cache, const at::Tensor &value_cache,
                          const PageTable &pages, const at::Tensor &seq_lens, const at::Tensor &partial_output,
                          const at::Tensor &partial_max, const at::Tensor &partial_sum, const at::Tensor &output,
                          int64_t max_seq_len, int64_t split_size, std::optional<double> softmax_scale, int64_t q_len,
                          const std::optional<at::Tensor> &lse, int32_t kv_dtype,
                          const std::optional<at::Tensor> &tree_mask) {
  TORCH_CHECK(query.dim() == 3, "invalid query");
  TORCH_CHECK(key_cache.dim() == 4 && key_cache.size(3) == query.size(2), "NHD cache only");
  TORCH_CHECK(key_cache.sizes() == value_cache.sizes(), "K/V cache mismatch");
  TORCH_CHECK(pages.table->scalar_type() == at::kInt, pages.indptr ? "int32 page indices" : "int32 block table");
  TORCH_CHECK(seq_lens.scalar_type() == at::kInt, "int32 sequence lengths");
  TORCH_CHECK(q_len >= 1, "q_len must be >= 1");
  TORCH_CHECK(query.size(1) % key_cache.size(2) == 0, "Q heads must be divisible by KV heads");
  TORCH_CHECK(query.size(0) % q_len == 0, "query rows must be batch * q_len");
  const int64_t rows = query.size(0);
  const int64_t batch = rows / q_len;
  const int64_t heads = query.size(1);
  const int64_t head_dim = query.size(2);
  if (pages.indptr) {
    const at::Tensor &ip = *pages.indptr;
    TORCH_CHECK(ip.scalar_type() == at::kInt && ip.dim() == 1 && ip.size(0) == batch + 1 && ip.is_contiguous(),
                "page_indptr must be contiguous int32 [batch + 1]");
    TORCH_CHECK(pages.table->dim() == 1 && pages.table->is_contiguous(), "page_indices must be contiguous 1-D");
    check_same_device(ip, query, "page_indptr");
  } else {
    TORCH_CHECK(pages.table->dim() == 2 && pages.table->size(0) == batch, "block table must be [batch, max_pages]");
    TORCH_CHECK(pages.table->stride(1) == 1, "block table rows and seq_lens must be contiguous");
  }
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.size(0) == batch, "seq_lens must be [batch]");
  TORCH_CHECK(seq_lens.is_contiguous(), "block table rows and seq_lens must be contiguous");
  TORCH_CHECK(output.sizes() == query.sizes() && output.scalar_type() == query.scalar_type(),
              "output must match the query's shape and dtype");
  for (const at::Tensor *t : {&key_cache, &value_cache, pages.table, &seq_lens, &output})
    check_same_device(*t, query, "every tensor");
  TORCH_CHECK(query.stride(2) == 1 && key_cache.stride(3) == 1 && value_cache.stride(3) == 1 &&
                  output.stride(2) == 1,
              "head_dim must be the contiguous dimension");
  const int64_t n_s = l20_pd_num_splits((int32_t)max_seq_len, (int32_t)split_size);
  const bool need_ws = n_s > 1;
  if (need_ws) {
    TORCH_CHECK(partial_output.dim() == 4 && partial_output.size(0) == rows && partial_output.size(1) == heads &&
                    partial_output.size(2) >= n_s && partial_output.size(3) == head_dim &&
                    partial_output.stride(3) == 1,
                "partial output workspace has wrong shape");
    TORCH_CHECK(partial_output.scalar_type() == at::kFloat || partial_output.scalar_type() == at::kHalf ||
                    partial_output.scalar_type() == at::kBFloat16,
                "partial output workspace must be fp32, fp16 or bf16");
    for (const at::Tensor *t : {&partial_max, &partial_sum}) {
      TORCH_CHECK(t->dim() == 3 && t->size(0) == rows && t->size(1) == heads && t->size(2) >= n_s &&
                      t->scalar_type() == at::kFloat,
                  "partial max/sum workspace has wrong shape");
      check_same_device(*t, query, "partial max/sum workspace");
    }
    check_same_device(partial_output, query, "partial output workspace");
  }
  float *lse_ptr = nullptr;
  int64_t lse_srow = 0, lse_shead = 0;
  if (lse.has_value() && lse->defined()) {
    const at::Tensor &t = *lse;
    TORCH_CHECK(t.scalar_type() == at::kFloat && t.dim() == 2 && t.size(0) == rows && t.size(1) == heads,
                "lse must be fp32 [batch*q_len, num_q_heads]");
    check_same_device(t, query, "lse");
    lse_ptr = t.data_ptr<float>();
    lse_srow = t.stride(0);
    lse_shead = t.stride(1);
  }

  l20_pd_fp8_args a{};
  a.query = query.data_ptr();
  a.query_dtype = dtype_code(query);
  a.q_stride_row = query.stride(0);
  a.q_stride_head = query.stride(1);
  a.key_cache = reinterpret_cast<const uint8_t *>(key_cache.data_ptr());
  a.k_stride_page = key_cache.stride(0);
  a.k_stride_token = key_cache.stride(1);
  a.k_stride_head = key_cache.stride(2);
  a.value_cache = reinterpret_cast<const uint8_t *>(value_cache.data_ptr());
  a.v_stride_page = value_cache.stride(0);
  a.v_stride_token = value_cache.stride(1);
  a.v_stride_head = value_cache.stride(2);
  a.num_pages = key_cache.size(0);
  a.page_size = (int32_t)key_cache.size(1);
  a.block_table = pages.table->data_ptr<int32_t>();
  if (pages.indptr) {
    a.page_indptr = pages.indptr->data_ptr<int32_t>();
  } else {
    a.bt_stride_row = pages.table->stride(0);
    a.bt_max_pages = (int32_t)pages.table->size(1);
  }
  a.seq_lens = seq_lens.data_ptr<int32_t>();
  if (need_ws) {
    a.partial_output = partial_output.data_ptr();
    a.partial_dtype = dtype_code(partial_output);
    a.po_stride_row = partial_output.stride(0);
    a.po_stride_head = partial_output.stride(1);
    a.po_stride_split = partial_output.stride(2);
    a.partial_splits = (int32_t)partial_output.size(2);
    a.partial_max = partial_max.data_ptr<float>();
    a.pm_stride_row = partial_max.stride(0);
    a.pm_stride_head = partial_max.stride(1);
    a.pm_stride_split = partial_max.stride(2);
    a.partial_sum = partial_sum.data_ptr<float>();
    a.ps_stride_row = partial_sum.stride(0);
    a.ps_stride_head = partial_sum.stride(1);
    a.ps_stride_split = partial_sum.stride(2);
  }
  a.output = output.data_ptr();
  a.o_stride_row = output.stride(0);
  a.o_stride_head = output.stride(1);
  a.lse = lse_ptr;
  a.lse_stride_row = lse_srow;
  a.lse_stride_head = lse_shead;
  a.k_scale = 1.0f;
  a.v_scale = 1.0f;
  a.softmax_scale = softmax_scale.has_value() ? (float)*softmax_scale : 0.0f;
  a.batch = (int32_t)batch;
  a.q_len = (int32_t)q_len;
  a.num_q_heads = (int32_t)heads;
  a.num_kv_heads = (int32_t)key_cache.size(2);
  a.head_dim = (int32_t)head_dim;
  a.max_seq_len = (int32_t)max_seq_len;
  a.split_size = (int32_t)split_size;
  a.kv_dtype = kv_dtype;
  if (tree_mask.has_value() && tree_mask->defined()) {
    const at::Tensor &t = *tree_mask;
    TORCH_CHECK(t.scalar_type() == at::kInt && t.size(-1) == q_len && t.stride(-1) == 1 &&
                    ((t.dim() == 1) || (t.dim() == 2 && t.size(0) == batch)),
                "tree_mask must be int32 [batch, q_len] or [q_len] ancestor bitmasks");
    check_same_device(t, query, "tree_mask");
    a.tree_mask = t.data_ptr<int32_t>();
    a.tree_mask_stride_batch = t.dim() == 2 ? t.stride(0) : 0;
  }
  return a;
}

void launch(const at::Tensor &query, const l20_pd_fp8_args &a, bool fp8) {
  const c10::DeviceGuard guard(query.device());
  void *stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.get_device()).stream();
  const int32_t rc = fp8 ? l20_pd_fp8_e4m3_split_out(&a, stream) : l20_pd_split_out(&a, stream);
  TORCH_CHECK(rc == L20_PD_OK, l20_pd_last_error());
}

void check_query(const at::Tensor &query) {
  TORCH_CHECK(query.is_cuda(), "query must be CUDA");
  TORCH_CHECK(query.scalar_type() == at::kBFloat16 || query.scalar_type() == at::kHalf,
              "query must be bf16 or fp16");
}

// 16-bit caches: the reference's fp16 op (FP16 only there); bf16 caches pair
// with a bf16 query.
int32_t check_16bit_cache(const at::Tensor &query, const at::Tensor &key_cache, const at::Tensor &value_cache) {
  TORCH_CHECK(key_cache.scalar_type() == query.scalar_type() && value_cache.scalar_type() == query.scalar_type(),
              "K/V cache must have the query's dtype (fp16 or bf16)");
  return query.scalar_type() == at::kBFloat16 ? L20_PD_KV_BF16 : L20_PD_KV_FP16;
}

at::Tensor paged_decode_fp8_e4m3_split_out(
    const at::Tensor &query, const at::Tensor &key_cache, const at::Tensor &value_cache,
    const at::Tensor &block_table, const at::Tensor &seq_lens, const at::Tensor &partial_output,
    const at::Tensor &partial_max, const at::Tensor &partial_sum, const at::Tensor &output, double k_scale,
    double v_scale, int64_t max_seq_len, int64_t split_size, std::optional<double> softmax_scale,
    const std::optional<at::Tensor> &k_scale_per_head, const std::optional<at::Tensor> &v_scale_per_head,
    int64_t q_len, const std::optional<at::Tensor> &lse, const std::optional<at::Tensor> &tree_mask) {
  check_query(query);
  // e4m3fn as in the reference's CUDA op; e5m2 as its Triton path accepts
  // (integrations/vllm/l20_paged_split_kv.py:617-621).
  const bool e5m2 = key_cache.scalar_type() == at::kFloat8_e5m2;
  TORCH_CHECK((key_cache.scalar_type() == at::kFloat8_e4m3fn || e5m2) &&
                  value_cache.scalar_type() == key_cache.scalar_type(),
              "K/V cache must be torch.float8_e4m3fn (or both torch.float8_e5m2)");
  l20_pd_fp8_args a = make_args(query, key_cache, value_cache, PageTable{&block_table, nullptr}, seq_lens,
                                partial_output, partial_max, partial_sum, output, max_seq_len, split_size,
                                softmax_scale, q_len, lse, e5m2 ? L20_PD_KV_FP8_E5M2 : L20_PD_KV_FP8_E4M3,
                                tree_mask);
  for (int which = 0; which < 2; ++which) {
    const auto &opt = which == 0 ? k_scale_per_head : v_scale_per_head;
    if (opt.has_value() && opt->defined()) {
      const at::Tensor &t = *opt;
      TORCH_CHECK(t.scalar_type() == at::kFloat && t.is_contiguous() && t.numel() == key_cache.size(2),
                  "per-head scales must be contiguous fp32 [num_kv_heads]");
      check_same_device(t, query, "per-head scales");
      (which == 0 ? a.k_scale_per_head : a.v_scale_per_head) = t.data_ptr<float>();
    }
  }
  a.k_scale = (float)k_scale;
  a.v_scale = (float)v_scale;
  launch(query, a, true);
  return output;
}

// l20_paged_decode_split_out_cuda (l20_paged_decode.cu:549-597).
at::Tensor paged_decode_split_out(const at::Tensor &query, const at::Tensor &key_cache, const at::Tensor &value_cache,
                                  const at::Tensor &block_table, const at::Tensor &seq_lens,
                                  const at::Tensor &partial_output, const at::Tensor &partial_max,
                                  const at::Tensor &partial_sum, const at::Tensor &output, int64_t max_seq_len,
                                  int64_t split_size, std::optional<double> softmax_scale, int64_t q_len,
                                  const std::optional<at::Tensor> &lse, const std::optional<at::Tensor> &tree_mask) {
  check_query(query);
  const int32_t kv = check_16bit_cache(query, key_cache, value_cache);
  const l20_pd_fp8_args a = make_args(query, key_cache, value_cache, PageTable{&block_table, nullptr}, seq_lens,
                                      partial_output, partial_max, partial_sum, output, max_seq_len, split_size,
                                      softmax_scale, q_len, lse, kv, tree_mask);
  launch(query, a, false);
  return output;
}

// l20_paged_decode_split_indices_out_cuda (l20_paged_decode.cu:600-649): CSR page list.
at::Tensor paged_decode_split_indices_out(const at::Tensor &query, const at::Tensor &key_cache,
                                          const at::Tensor &value_cache, const at::Tensor &page_indptr,
                                          const at::Tensor &page_indices, const at::Tensor &seq_lens,
                                          const at::Tensor &partial_output, const at::Tensor &partial_max,
                                          const at::Tensor &partial_sum, const at::Tensor &output,
                                          int64_t max_seq_len, int64_t split_size,
                                          std::optional<double> softmax_scale, int64_t q_len,
                                          const std::optional<at::Tensor> &lse,
                                          const std::optional<at::Tensor> &tree_mask) {
  check_query(query);
  const int32_t kv = check_16bit_cache(query, key_cache, value_cache);
  const l20_pd_fp8_args a = make_args(query, key_cache, value_cache, PageTable{&page_indices, &page_indptr},
                                      seq_lens, partial_output, partial_max, partial_sum, output, max_seq_len,
                                      split_size, softmax_scale, q_len, lse, kv, tree_mask);
  launch(query, a, false);
  return output;
}

// ---------------------------------------------------------------------------
// Paged KV-cache producer: l20_rope_and_cache (integrations/vllm/l20_rope_kv.py:256-309)
// with fp8 caches, and the fp8 scale helper.
// ---------------------------------------------------------------------------
l20_pd_kv_write_args kv_args(const std::optional<at::Tensor> &query, const at::Tensor &key, const at::Tensor &value,
                             const at::Tensor &positions, const at::Tensor &cos_sin_cache, bool is_neox,
                             const at::Tensor &key_cache, const at::Tensor &value_cache,
                             const at::Tensor &slot_mapping) {
  TORCH_CHECK(key.is_cuda(), "key must be CUDA");
  TORCH_CHECK(key.scalar_type() == at::kBFloat16 || key.scalar_type() == at::kHalf,
              "l20_rope_and_cache supports FP16 and BF16");
  TORCH_CHECK(value.scalar_type() == key.scalar_type(), "Q, K, and V must use the same dtype");
  TORCH_CHECK(key.dim() == 3 && value.dim() == 3, "Q, K, and V must be [tokens, heads, head_dim]");
  TORCH_CHECK(key.sizes() == value.sizes(), "Q, K, and V shapes are incompatible");
  const bool has_q = query.has_value() && query->defined();
  if (has_q) {
    TORCH_CHECK(query->scalar_type() == key.scalar_type(), "Q, K, and V must use the same dtype");
    TORCH_CHECK(query->dim() == 3 && query->size(0) == key.size(0) && query->size(2) == key.size(2),
                "Q, K, and V shapes are incompatible");
    TORCH_CHECK(query->stride(2) == 1, "head_dim must be the contiguous dimension");
    check_same_device(*query, key, "query");
  }
  TORCH_CHECK(key_cache.dim() == 4 && value_cache.sizes() == key_cache.sizes(),
              "cache must use NHD [blocks, block, heads, dim]");
  // Pages of any multiple of 16 tokens; a page of 16 m tokens is written as m
  // 16-token sub-pages (slot s is sub-page s / 16, row s % 16), which needs
  // its tokens contiguous.
  const int64_t page_tokens = key_cache.size(1);
  TORCH_CHECK(page_tokens >= 16 && page_tokens % 16 == 0, "cache block size must be a multiple of 16");
  TORCH_CHECK(page_tokens == 16 || (key_cache.stride(0) == page_tokens * key_cache.stride(1) &&
                                    value_cache.stride(0) == page_tokens * value_cache.stride(1)),
              "cache blocks of more than 16 tokens must hold them contiguously");
  TORCH_CHECK(key_cache.size(2) == key.size(1) && key_cache.size(3) == key.size(2),
              "cache head shape must match K/V");
  const bool fp8 = key_cache.scalar_type() == at::kFloat8_e4m3fn;
  TORCH_CHECK(fp8 || key_cache.scalar_type() == key.scalar_type(),
              "K/V cache must be torch.float8_e4m3fn or the model dtype");
  TORCH_CHECK(value_cache.scalar_type() == key_cache.scalar_type(), "K/V cache mismatch");
  TORCH_CHECK(positions.scalar_type() == at::kLong && slot_mapping.scalar_type() == at::kLong,
              "positions and slot_mapping must be int64");
  TORCH_CHECK(positions.numel() == key.size(0) && slot_mapping.numel() == key.size(0),
              "positions and slot_mapping must match token count");
  TORCH_CHECK(positions.is_contiguous() && slot_mapping.is_contiguous(), "positions and slot_mapping must be contiguous");
  TORCH_CHECK(cos_sin_cache.dim() == 2 && cos_sin_cache.stride(1) == 1, "invalid cos_sin_cache rotary dimension");
  const int64_t rot = cos_sin_cache.size(1);
  TORCH_CHECK(rot > 0 && rot <= key.size(2) && rot % 2 == 0, "invalid cos_sin_cache rotary dimension");
  for (const at::Tensor *t : {&value, &positions, &cos_sin_cache, &key_cache, &value_cache, &slot_mapping})
    check_same_device(*t, key, "every tensor");
  TORCH_CHECK(key.stride(2) == 1 && value.stride(2) == 1 && key_cache.stride(3) == 1 && value_cache.stride(3) == 1,
              "head_dim must be the contiguous dimension");
  l20_pd_kv_write_args a{};
  if (has_q) {
    a.query = query->data_ptr();
    a.q_stride_token = query->stride(0);
    a.q_stride_head = query->stride(1);
    a.num_q_heads = (int32_t)query->size(1);
  }
  a.key = key.data_ptr();
  a.k_stride_token = key.stride(0);
  a.k_stride_head = key.stride(1);
  a.value = value.data_ptr();
  a.v_stride_token = value.stride(0);
  a.v_stride_head = value.stride(1);
  a.dtype = dtype_code(key);
  a.positions = positions.data_ptr<int64_t>();
  a.cos_sin_cache = cos_sin_cache.data_ptr();
  a.cs_stride_position = cos_sin_cache.stride(0);
  a.cs_dtype = dtype_code(cos_sin_cache);
  a.rotary_dim = (int32_t)rot;
  a.is_neox = is_neox ? 1 : 0;
  a.slot_mapping = slot_mapping.data_ptr<int64_t>();
  a.key_cache = key_cache.data_ptr();
  a.kc_stride_page = page_tokens == 16 ? key_cache.stride(0) : 16 * key_cache.stride(1);
  a.kc_stride_token = key_cache.stride(1);
  a.kc_stride_head = key_cache.stride(2);
  a.value_cache = value_cache.data_ptr();
  a.vc_stride_page = page_tokens == 16 ? value_cache.stride(0) : 16 * value_cache.stride(1);
  a.vc_stride_token = value_cache.stride(1);
  a.vc_stride_head = value_cache.stride(2);
  a.num_pages = key_cache.size(0) * (page_tokens / 16);
  a.cache_dtype = fp8 ? L20_PD_KV_FP8_E4M3 : (key.scalar_type() == at::kBFloat16 ? L20_PD_KV_BF16 : L20_PD_KV_FP16);
  a.k_scale = 1.0f;
  a.v_scale = 1.0f;
  a.num_tokens = (int32_t)key.size(0);
  a.num_kv_heads = (int32_t)key.size(1);
  a.head_dim = (int32_t)key.size(2);
  return a;
}

const float *per_head_scale(const std::optional<at::Tensor> &t, const at::Tensor &key) {
  if (!t.has_value() || !t->defined()) return nullptr;
  TORCH_CHECK(t->scalar_type() == at::kFloat && t->is_contiguous() && t->numel() == key.size(1),
              "per-head scales must be contiguous fp32 [num_kv_heads]");
  check_same_device(*t, key, "per-head scales");
  return t->data_ptr<float>();
}

void rope_and_cache(const std::optional<at::Tensor> &query, const at::Tensor &key, const at::Tensor &value,
                    const at::Tensor &positions, const at::Tensor &cos_sin_cache, bool is_neox,
                    const at::Tensor &key_cache, const at::Tensor &value_cache, const at::Tensor &slot_mapping,
                    double k_scale, double v_scale, const std::optional<at::Tensor> &k_scale_per_head,
                    const std::optional<at::Tensor> &v_scale_per_head) {
  l20_pd_kv_write_args a =
      kv_args(query, key, value, positions, cos_sin_cache, is_neox, key_cache, value_cache, slot_mapping);
  a.k_scale = (float)k_scale;
  a.v_scale = (float)v_scale;
  a.k_scale_per_head = per_head_scale(k_scale_per_head, key);
  a.v_scale_per_head = per_head_scale(v_scale_per_head, key);
  const c10::DeviceGuard guard(key.device());
  void *stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  const int32_t rc = l20_pd_rope_and_cache(&a, stream);
  TORCH_CHECK(rc == L20_PD_OK, l20_pd_last_error());
}

void kv_fp8_scales(const at::Tensor &key, const at::Tensor &value, const at::Tensor &positions,
                   const at::Tensor &cos_sin_cache, bool is_neox, const at::Tensor &key_cache,
                   const at::Tensor &value_cache, const at::Tensor &slot_mapping, const at::Tensor &k_scales,
                   const at::Tensor &v_scales, bool per_head) {
  const l20_pd_kv_write_args a =
      kv_args(std::nullopt, key, value, positions, cos_sin_cache, is_neox, key_cache, value_cache, slot_mapping);
  for (const at::Tensor *t : {&k_scales, &v_scales}) {
    TORCH_CHECK(t->scalar_type() == at::kFloat && t->is_contiguous() && t->numel() == key.size(1),
                "scale outputs must be contiguous fp32 [num_kv_heads]");
    check_same_device(*t, key, "scale outputs");
  }
  const c10::DeviceGuard guard(key.device());
  void *stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  const int32_t rc =
      l20_pd_kv_fp8_scales(&a, k_scales.data_ptr<float>(), v_scales.data_ptr<float>(), per_head ? 1 : 0, stream);
  TORCH_CHECK(rc == L20_PD_OK, l20_pd_last_error());
}

// Draft-suffix attention merged with the paged prefix's result (the suffix and
// merge launches of src/l20_stack/ops/triton_tree_attention.py:1152-1197).
void tree_suffix_merge(const at::Tensor &query, const at::Tensor &suffix_key, const at::Tensor &suffix_value,
                       const at::Tensor &ancestor_mask, const at::Tensor &prefix_output,
                       const at::Tensor &prefix_lse, const at::Tensor &output, double softmax_scale) {
  check_query(query);
  TORCH_CHECK(query.dim() == 4, "expected query=[B,S,Hq,D]");
  TORCH_CHECK(suffix_key.dim() == 4 && suffix_value.sizes() == suffix_key.sizes(),
              "expected suffix key/value=[B,S,Hkv,D]");
  TORCH_CHECK(suffix_key.scalar_type() == query.scalar_type() && suffix_value.scalar_type() == query.scalar_type(),
              "suffix key/value must have the query's dtype");
  TORCH_CHECK(suffix_key.size(0) == query.size(0) && suffix_key.size(1) == query.size(1) &&
                  suffix_key.size(3) == query.size(3),
              "suffix KV must match query batch/draft and cache kv heads");
  TORCH_CHECK(ancestor_mask.dim() == 2 && ancestor_mask.size(0) == query.size(1) &&
                  ancestor_mask.size(1) == query.size(1) &&
                  (ancestor_mask.scalar_type() == at::kBool || ancestor_mask.scalar_type() == at::kByte),
              "ancestor_mask must match draft_length");
  TORCH_CHECK(prefix_output.sizes() == query.sizes() && output.sizes() == query.sizes(),
              "prefix_output and output must be shaped like the query");
  TORCH_CHECK(output.scalar_type() == query.scalar_type(), "output must have the query's dtype");
  TORCH_CHECK(prefix_lse.scalar_type() == at::kFloat && prefix_lse.dim() == 3 &&
                  prefix_lse.size(0) == query.size(0) && prefix_lse.size(1) == query.size(1) &&
                  prefix_lse.size(2) == query.size(2),
              "prefix_lse must be fp32 [B,S,Hq]");
  for (const at::Tensor *t : {&query, &suffix_key, &suffix_value, &prefix_output, &output})
    TORCH_CHECK(t->stride(3) == 1, "head_dim must be the contiguous dimension");
  for (const at::Tensor *t : {&suffix_key, &suffix_value, &ancestor_mask, &prefix_output, &prefix_lse, &output})
    check_same_device(*t, query, "every tensor");
  l20_pd_tree_suffix_args a{};
  a.query = query.data_ptr();
  a.q_stride_batch = query.stride(0);
  a.q_stride_draft = query.stride(1);
  a.q_stride_head = query.stride(2);
  a.query_dtype = dtype_code(query);
  a.suffix_key = suffix_key.data_ptr();
  a.sk_stride_batch = suffix_key.stride(0);
  a.sk_stride_draft = suffix_key.stride(1);
  a.sk_stride_head = suffix_key.stride(2);
  a.suffix_value = suffix_value.data_ptr();
  a.sv_stride_batch = suffix_value.stride(0);
  a.sv_stride_draft = suffix_value.stride(1);
  a.sv_stride_head = suffix_value.stride(2);
  a.ancestor_mask = static_cast<const uint8_t *>(ancestor_mask.data_ptr());
  a.mask_stride_row = ancestor_mask.stride(0);
  a.mask_stride_col = ancestor_mask.stride(1);
  a.prefix_output = prefix_output.data_ptr();
  a.po_stride_batch = prefix_output.stride(0);
  a.po_stride_draft = prefix_output.stride(1);
  a.po_stride_head = prefix_output.stride(2);
  a.prefix_dtype = dtype_code(prefix_output);
  a.prefix_lse = prefix_lse.data_ptr<float>();
  a.pl_stride_batch = prefix_lse.stride(0);
  a.pl_stride_draft = prefix_lse.stride(1);
  a.pl_stride_head = prefix_lse.stride(2);
  a.output = output.data_ptr();
  a.o_stride_batch = output.stride(0);
  a.o_stride_draft = output.stride(1);
  a.o_stride_head = output.stride(2);
  a.softmax_scale = (float)softmax_scale;
  a.batch = (int32_t)query.size(0);
  a.draft_length = (int32_t)query.size(1);
  a.num_q_heads = (int32_t)query.size(2);
  a.num_kv_heads = (int32_t)suffix_key.size(2);
  a.head_dim = (int32_t)query.size(3);
  const c10::DeviceGuard guard(query.device());
  void *stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.get_device()).stream();
  const int32_t rc = l20_pd_tree_suffix_merge(&a, stream);
  TORCH_CHECK(rc == L20_PD_OK, l20_pd_last_error());
}

}  // namespace

TORCH_LIBRARY(l20_stack, m) {
  m.def(
      "paged_decode_split_out("
      "Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, Tensor seq_lens, "
      "Tensor(a!) partial_output, Tensor(b!) partial_max, "
      "Tensor(c!) partial_sum, Tensor(d!) output, "
      "int max_seq_len, int split_size, "
      "float? softmax_scale=None, int q_len=1, "
      "Tensor(e!)? lse=None, Tensor? tree_mask=None) -> Tensor(d!)");
  m.def(
      "paged_decode_fp8_e4m3_split_out("
      "Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, Tensor seq_lens, "
      "Tensor(a!) partial_output, Tensor(b!) partial_max, "
      "Tensor(c!) partial_sum, Tensor(d!) output, "
      "float k_scale, float v_scale, "
      "int max_seq_len, int split_size, "
      "float? softmax_scale=None, Tensor? k_scale_per_head=None, "
      "Tensor? v_scale_per_head=None, int q_len=1, "
      "Tensor(e!)? lse=None, Tensor? tree_mask=None) -> Tensor(d!)");
  m.def(
      "paged_decode_split_indices_out("
      "Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor page_indptr, Tensor page_indices, Tensor seq_lens, "
      "Tensor(a!) partial_output, Tensor(b!) partial_max, "
      "Tensor(c!) partial_sum, Tensor(d!) output, "
      "int max_seq_len, int split_size, "
      "float? softmax_scale=None, int q_len=1, "
      "Tensor(e!)? lse=None, Tensor? tree_mask=None) -> Tensor(d!)");
  m.def(
      "rope_and_cache(Tensor(a!)? query, Tensor(b!) key, Tensor value, Tensor positions, "
      "Tensor cos_sin_cache, bool is_neox, Tensor(c!) key_cache, Tensor(d!) value_cache, "
      "Tensor slot_mapping, float k_scale=1.0, float v_scale=1.0, "
      "Tensor? k_scale_per_head=None, Tensor? v_scale_per_head=None) -> ()");
  m.def(
      "kv_fp8_scales(Tensor key, Tensor value, Tensor positions, Tensor cos_sin_cache, bool is_neox, "
      "Tensor key_cache, Tensor value_cache, Tensor slot_mapping, Tensor(a!) k_scales, "
      "Tensor(b!) v_scales, bool per_head=True) -> ()");
  m.def(
      "tree_suffix_merge(Tensor query, Tensor suffix_key, Tensor suffix_value, Tensor ancestor_mask, "
      "Tensor prefix_output, Tensor prefix_lse, Tensor(a!) output, float softmax_scale) -> ()");
}

TORCH_LIBRARY_IMPL(l20_stack, CUDA, m) {
  m.impl("rope_and_cache", &rope_and_cache);
  m.impl("kv_fp8_scales", &kv_fp8_scales);
  m.impl("paged_decode_split_out", &paged_decode_split_out);
  m.impl("paged_decode_fp8_e4m3_split_out", &paged_decode_fp8_e4m3_split_out);
  m.impl("paged_decode_split_indices_out", &paged_decode_split_indices_out);
  m.impl("tree_suffix_merge", &tree_suffix_merge);
}
