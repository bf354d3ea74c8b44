/*
 * C ABI of the paged KV-cache producer in libl20_paged_decode_hip.so:
 * rotary embedding of Q and K, and the paged write of K and V into fp8
 * (OCP e4m3fn) or 16-bit caches.  Plain pointers, sizes and strides; a HIP
 * stream is passed as `void *`.
 *
 * Reference interfaces replaced (paths relative to the reference repo root):
 *   l20_pd_rope_and_cache  <- l20_rope_and_cache, integrations/vllm/l20_rope_kv.py:256-309
 *                             (kernels :26-137 interleaved, :140-253 neox), which writes
 *                             16-bit caches only ("quantized KV cache is not supported",
 *                             :276-277); here fp8 caches are written with the quantiser
 *                             of scripts/smoke_cuda_paged_fp8_decode_op.py:13-19
 *   l20_pd_kv_fp8_scales   <- the scale rule of the same quantiser,
 *                             scale = max(amax / 448, 1e-12), per tensor or per KV head
 */
#ifndef L20_KV_WRITE_H_
#define L20_KV_WRITE_H_

#include <stdint.h>

#include "l20_paged_decode.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * One rope-and-cache call over num_tokens new tokens.  Strides are in
 * elements; head_dim is contiguous everywhere.
 *
 *   query          [num_tokens, num_q_heads, head_dim] dtype, rotated in place (NULL: skipped)
 *   key            [num_tokens, num_kv_heads, head_dim] dtype, rotated in place
 *   value          [num_tokens, num_kv_heads, head_dim] dtype
 *   positions      [num_tokens] int64 rotary positions
 *   cos_sin_cache  [max_position, rotary_dim] cs_dtype: cos in the first half, sin in the second
 *   slot_mapping   [num_tokens] int64: cache page slot // 16, row slot % 16; < 0 skips the token
 *   key/value_cache[num_pages, 16, num_kv_heads, head_dim] cache_dtype (enum l20_pd_kv_dtype;
 *                  a 16-bit cache must have the model dtype).  A cache of P-token pages
 *                  (P a multiple of 16, tokens contiguous) is passed as its 16-token
 *                  sub-pages: num_pages * P / 16 pages, stride_page = 16 * stride_token;
 *                  slot s (page s // P, row s % P) is then sub-page s // 16, row s % 16
 *
 * x' = x cos + (x_pair sin) sign on the first rotary_dim dims (each product
 * and the sum rounded to fp32, the result rounded to dtype), pairs
 * (d, d + rotary_dim/2) with is_neox, (2i, 2i+1) without.  fp8 caches store
 * RNE_e4m3fn(clamp(x / scale, +-448)) of the stored model-dtype values, with
 * the per-head scale arrays (fp32 [num_kv_heads], device memory) when
 * non-NULL, else the scalar scales.
 */
typedef struct l20_pd_kv_write_args {
  void *query;
  int64_t q_stride_token, q_stride_head;
  int32_t num_q_heads;
  void *key;
  int64_t k_stride_token, k_stride_head;
  const void *value;
  int64_t v_stride_token, v_stride_head;
  int32_t dtype; /* L20_PD_BF16 or L20_PD_FP16: query, key and value */

  const int64_t *positions;
  const void *cos_sin_cache;
  int64_t cs_stride_position;
  int32_t cs_dtype; /* L20_PD_BF16, L20_PD_FP16 or L20_PD_FP32 */
  int32_t rotary_dim;
  int32_t is_neox;

  const int64_t *slot_mapping;
  void *key_cache;
  int64_t kc_stride_page, kc_stride_token, kc_stride_head;
  void *value_cache;
  int64_t vc_stride_page, vc_stride_token, vc_stride_head;
  int64_t num_pages;
  int32_t cache_dtype; /* enum l20_pd_kv_dtype */

  float k_scale, v_scale;
  const float *k_scale_per_head;
  const float *v_scale_per_head;

  int32_t num_tokens, num_kv_heads, head_dim;
} l20_pd_kv_write_args;

/* Validate without touching the GPU: L20_PD_OK or L20_PD_EINVAL (message in
 * l20_pd_last_error()).  head_dim a multiple of 4 up to 256, rotary_dim a
 * multiple of 8 up to head_dim. */
int32_t l20_pd_kv_write_check(const l20_pd_kv_write_args *args);

/* Rotate Q and K in place and write K and V to the paged caches. */
int32_t l20_pd_rope_and_cache(const l20_pd_kv_write_args *args, void *stream);

/* Scales for an fp8 cache from the values rope_and_cache would store (the
 * rotated, dtype-rounded K and the V rows of `args`; nothing is written but
 * the outputs): k_scales / v_scales [num_kv_heads] fp32 device arrays receive
 * max(amax / 448, 1e-12) per head, or with per_head = 0 the per-tensor scale
 * in every entry. */
int32_t l20_pd_kv_fp8_scales(const l20_pd_kv_write_args *args, float *k_scales, float *v_scales,
                             int32_t per_head, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* L20_KV_WRITE_H_ */
