/*
 * C ABI of the draft-suffix step of hybrid tree attention in
 * libl20_paged_decode_hip.so: attention of each draft row over the
 * contiguous draft keys it may see, merged with the row's attention over
 * the paged prefix.  Plain pointers, element strides (head_dim contiguous
 * everywhere) and a HIP stream passed as `void *`.
 *
 * Reference interfaces replaced (paths relative to the reference repo root):
 *   l20_pd_tree_suffix_merge <- the suffix-summary and summary-merge launches of
 *                               hybrid_tree_attention_paged_prefix,
 *                               src/l20_stack/ops/triton_tree_attention.py:1152-1197
 *                               (kernels _tree_suffix_summary_kernel :436-510 and
 *                               _tree_summary_merge_kernel :513-545), fused into one
 *                               launch that reads the prefix pass's normalised
 *                               output and natural-log LSE.
 */
#ifndef L20_TREE_VERIFY_H_
#define L20_TREE_VERIFY_H_

#include <stdint.h>

#include "l20_paged_decode.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 *   query         [batch, draft, num_q_heads, head_dim] query_dtype
 *   suffix_key    [batch, draft, num_kv_heads, head_dim] query_dtype (draft token j of
 *                 sequence b at [b, j])
 *   suffix_value  same layout as suffix_key
 *   ancestor_mask [draft, draft] bytes: row i sees draft j iff mask[i][j] != 0 (a torch
 *                 bool tensor's storage)
 *   prefix_output [batch, draft, num_q_heads, head_dim] prefix_dtype: softmax-normalised
 *                 attention of each row over the prefix
 *   prefix_lse    [batch, draft, num_q_heads] fp32 natural-log LSE of the prefix scores
 *                 (-inf: no prefix key; prefix_output is then not read)
 *   output        [batch, draft, num_q_heads, head_dim] query_dtype; may be the same
 *                 memory as prefix_output (same dtype and strides)
 *
 * Row (b, i, h) with KV head h / (num_q_heads / num_kv_heads) computes, in fp32,
 * s_j = softmax_scale * q . k_j over the visible drafts j and
 *   out = (e^lse o_prefix + sum_j e^s_j v_j) / (e^lse + sum_j e^s_j),
 * the LSE merge of the reference's _tree_summary_merge_kernel.  A row with no
 * visible key at all is written as zeros.
 */
typedef struct l20_pd_tree_suffix_args {
  const void *query;
  int64_t q_stride_batch, q_stride_draft, q_stride_head;
  int32_t query_dtype; /* L20_PD_BF16 or L20_PD_FP16 */
  const void *suffix_key;
  int64_t sk_stride_batch, sk_stride_draft, sk_stride_head;
  const void *suffix_value;
  int64_t sv_stride_batch, sv_stride_draft, sv_stride_head;
  const uint8_t *ancestor_mask;
  int64_t mask_stride_row, mask_stride_col;
  const void *prefix_output;
  int64_t po_stride_batch, po_stride_draft, po_stride_head;
  int32_t prefix_dtype; /* query_dtype or L20_PD_FP32 */
  const float *prefix_lse;
  int64_t pl_stride_batch, pl_stride_draft, pl_stride_head;
  void *output;
  int64_t o_stride_batch, o_stride_draft, o_stride_head;
  float softmax_scale;
  int32_t batch, draft_length, num_q_heads, num_kv_heads, head_dim;
} l20_pd_tree_suffix_args;

/* Validate without touching the GPU (draft_length 1..64, head_dim 64 or 128,
 * integral GQA ratio, non-null pointers, known dtypes). */
int32_t l20_pd_tree_suffix_check(const l20_pd_tree_suffix_args *args);

/* Enqueue the suffix attention + merge on `stream`; allocates nothing.  One wave
 * per (sequence, draft row, query head). */
int32_t l20_pd_tree_suffix_merge(const l20_pd_tree_suffix_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* L20_TREE_VERIFY_H_ */
