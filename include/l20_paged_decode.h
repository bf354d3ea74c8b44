/*
 * C ABI of the MI355X (gfx950) paged FP8-KV decode-attention library
 * (libl20_paged_decode_hip.so).
 *
 * Every entry point takes plain pointers, sizes and strides; no torch or HIP
 * types appear in the signatures (a HIP stream is passed as `void *`).  The
 * torch binding (l20_paged_decode_ops.so, TORCH_LIBRARY(l20_stack)) and the
 * ctypes binding used by the tests both call through these functions.
 *
 * Reference interfaces replaced (paths relative to the reference repo root):
 *   l20_pd_fp8_e4m3_split_out  <- l20_paged_decode_fp8_e4m3_split_out_cuda
 *                                 integrations/vllm/cuda/l20_paged_decode.cu:651-725
 *                                 (declared at l20_paged_decode.cpp:47-60, bound by
 *                                 TORCH_LIBRARY(l20_stack) at l20_paged_decode.cpp:128-143)
 *   l20_pd_fp8_e4m3_check      <- the TORCH_CHECK block of the same function,
 *                                 l20_paged_decode.cu:665-688 (argument validation
 *                                 without touching the GPU)
 *   l20_pd_num_splits          <- num_splits = ceil(max_seq_len / split_size),
 *                                 l20_paged_decode.cu:684
 *   l20_pd_fp8_e4m3_dequant_f32/_bf16
 *                              <- fp8x2_e4m3fn_to_float2, l20_paged_decode.cu:20-33
 *                                 (the device-side e4m3fn conversion, exposed as a
 *                                 bulk dequantiser)
 *   l20_pd_split_out           <- l20_paged_decode_split_out_cuda (fp16 caches,
 *                                 l20_paged_decode.cu:549-597, TORCH_LIBRARY schema at
 *                                 l20_paged_decode.cpp:121-127) and
 *                                 l20_paged_decode_split_indices_out_cuda (CSR page
 *                                 lists, l20_paged_decode.cu:600-649, pybind export at
 *                                 l20_paged_decode.cpp:150-152)
 */
#ifndef L20_PAGED_DECODE_H_
#define L20_PAGED_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define L20_PD_ABI_VERSION 4

/* Element types for query/output and the partial-output workspace. */
enum l20_pd_dtype {
  L20_PD_BF16 = 0,
  L20_PD_FP16 = 1,
  L20_PD_FP32 = 2
};

/* Element types of the K/V caches. */
enum l20_pd_kv_dtype {
  L20_PD_KV_FP8_E4M3 = 0,  /* OCP e4m3fn codes, dequantised as code * scale */
  L20_PD_KV_FP16 = 1,      /* fp16 values (query must be fp16) */
  L20_PD_KV_BF16 = 2,      /* bf16 values (query must be bf16) */
  L20_PD_KV_FP8_E5M2 = 3   /* OCP e5m2 codes, dequantised as code * scale (the fp8 entry
                              points; the reference's hook-facing Triton path accepts
                              torch.float8_e5m2 caches, integrations/vllm/l20_paged_split_kv.py:617-621) */
};

/* Return codes. */
enum l20_pd_status {
  L20_PD_OK = 0,
  L20_PD_EINVAL = 1,   /* argument validation failed; see l20_pd_last_error() */
  L20_PD_ELAUNCH = 2   /* a HIP launch or runtime call failed */
};

/*
 * Arguments of one paged FP8 decode-attention call.  Strides are in elements
 * of the tensor's own type (bytes for the fp8 caches).  The last dimension of
 * every tensor (head_dim) must be contiguous.
 *
 *   query          [batch*q_len, num_q_heads, head_dim]   bf16 or fp16
 *   key/value      [num_pages, page_size, num_kv_heads, head_dim]  e4m3fn bytes; page_size
 *                  any multiple of 16 through 4096 (above 16 a page's tokens must be
 *                  contiguous: stride_page = page_size * stride_token); token t of a
 *                  sequence is row t % page_size of page block_table[b][t / page_size]
 *   block_table    [batch, >= ceil(max_seq_len/page_size)]  int32 physical page ids, or,
 *                  with page_indptr [batch+1] (CSR), the flat page list: sequence b's
 *                  pages are block_table[page_indptr[b] .. page_indptr[b+1])
 *   seq_lens       [batch]  int32, each <= max_seq_len, includes the q_len new tokens
 *   partial_output [batch*q_len, num_q_heads, >= num_splits, head_dim]  fp32, fp16 or bf16
 *                  (bf16: what the reference's hook-facing allocator gives a bf16 query,
 *                  integrations/vllm/l20_paged_split_kv.py:24-26)
 *   partial_max/sum[batch*q_len, num_q_heads, >= num_splits]  fp32
 *   output         [batch*q_len, num_q_heads, head_dim]  same dtype as query
 *   lse            [batch*q_len, num_q_heads] fp32 natural-log LSE, or NULL
 *
 * Query row b*q_len+i attends to keys 0 .. seq_lens[b]-q_len+i (causal among
 * the q_len newest tokens; q_len=1 is plain decode).  K/V are dequantised as
 * code * scale with the per-head scale arrays (fp32 [num_kv_heads], device
 * memory) when non-NULL, else with the scalar scales.  softmax_scale <= 0
 * selects head_dim^-0.5.  The contents of the partial workspace after a call
 * are unspecified.  kv_dtype selects the cache element type (strides of
 * 16-bit caches are in elements, like every other tensor); a zero-initialised
 * struct describes fp8 caches addressed through a block table.
 */
typedef struct l20_pd_fp8_args {
  const void *query;
  int32_t query_dtype;
  int64_t q_stride_row, q_stride_head;

  const uint8_t *key_cache;
  int64_t k_stride_page, k_stride_token, k_stride_head;
  const uint8_t *value_cache;
  int64_t v_stride_page, v_stride_token, v_stride_head;
  int64_t num_pages;
  int32_t page_size;

  const int32_t *block_table;
  int64_t bt_stride_row;
  int32_t bt_max_pages;
  const int32_t *seq_lens;

  void *partial_output;
  int32_t partial_dtype;
  int64_t po_stride_row, po_stride_head, po_stride_split;
  int32_t partial_splits;
  float *partial_max;
  int64_t pm_stride_row, pm_stride_head, pm_stride_split;
  float *partial_sum;
  int64_t ps_stride_row, ps_stride_head, ps_stride_split;

  void *output;
  int64_t o_stride_row, o_stride_head;
  float *lse;
  int64_t lse_stride_row, lse_stride_head;

  float k_scale, v_scale;
  const float *k_scale_per_head;
  const float *v_scale_per_head;
  float softmax_scale;

  int32_t batch, q_len, num_q_heads, num_kv_heads, head_dim;
  int32_t max_seq_len, split_size;

  /* ABI version 2 */
  int32_t kv_dtype;                /* enum l20_pd_kv_dtype */
  const int32_t *page_indptr;      /* CSR row offsets [batch+1], or NULL for block_table rows */

  /* ABI version 3: tree (ancestor-mask) verification.  tree_mask[b * stride + i]
   * (int32, bit j) lets query row b*q_len+i see key seq_lens[b]-q_len+j; the keys
   * before the newest q_len stay visible to every row.  NULL keeps the causal
   * rule (row i sees those keys up to its own).  stride 0 shares one mask. */
  const int32_t *tree_mask;
  int64_t tree_mask_stride_batch;
} l20_pd_fp8_args;

/* ABI version of the loaded library (L20_PD_ABI_VERSION). */
int32_t l20_pd_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *l20_pd_last_error(void);

/* ceil(max_seq_len / split_size); 0 for max_seq_len <= 0. */
int32_t l20_pd_num_splits(int32_t max_seq_len, int32_t split_size);

/* Validate `args` exactly as l20_pd_fp8_e4m3_split_out does, without any
 * HIP call.  Returns L20_PD_OK or L20_PD_EINVAL. */
int32_t l20_pd_fp8_e4m3_check(const l20_pd_fp8_args *args);

/* Enqueue the split-KV partial kernel and the LSE merge kernel on `stream`
 * (hipStream_t, NULL = default stream).  Asynchronous; allocates nothing.
 * Requires kv_dtype == L20_PD_KV_FP8_E4M3.  Calls on different streams of one
 * device may overlap (each with its own workspace and output): the partial
 * kernel's work-queue counters (64 slots per device) are given per stream --
 * calls on one stream run in order and share its slot, up to 48 streams get
 * slots of their own (least recently used ones are shared beyond that), and a
 * call captured into a HIP graph takes one of 16 further slots in turn, since
 * the graph may replay on any stream.  Two launches that overlap in time on
 * one slot (a 49th stream in use at once, one graph replayed on two streams
 * at once, or two graphs captured 16 captures apart replayed at once) are
 * reported through l20_pd_device_errors (L20_PD_DEVERR_QUEUE_SHARED) whenever
 * their claims interleave; a launch that claims nothing shares nothing.
 * (<- l20_paged_decode_fp8_e4m3_split_out_cuda, l20_paged_decode.cu:651-725) */
int32_t l20_pd_fp8_e4m3_split_out(const l20_pd_fp8_args *args, void *stream);

/* Device-side errors of the partial kernel (no counterpart in the reference,
 * whose kernels have no inter-wave waits).  Its hand-off waits between the
 * waves of a workgroup give up after ~0.1 s of polling instead of hanging;
 * the wave records one of these codes and exits normally (its results are
 * then incomplete).  Returns the bitwise OR of the codes recorded on the
 * current device since the last clear (0: none), or -L20_PD_ELAUNCH on a HIP
 * error.  Synchronizes the device.  clear != 0 zeroes the error words and
 * the work-queue counters of every slot; call it only while no call of this
 * library is in flight. */
#define L20_PD_DEVERR_PREFIX_WAIT 1   /* the per-sequence item table was never published */
#define L20_PD_DEVERR_ACK_WAIT 2      /* a wave never acknowledged the published item */
#define L20_PD_DEVERR_PUBLISH_WAIT 4  /* the next item was never published */
#define L20_PD_DEVERR_QUEUE_SHARED 32 /* a work-queue claim found the counter in use by
                                         another launch: two launches overlapped on one
                                         slot (see l20_pd_fp8_e4m3_split_out), or one that
                                         gave up left it mid-way.  The workgroup stops
                                         claiming, so this launch's results (and the
                                         other's) may be incomplete, and the slot stays
                                         flagged until cleared: synchronize, clear, and
                                         repeat the calls */
int32_t l20_pd_device_errors(int32_t clear);

/* Polls before a hand-off wait gives up, for calls enqueued on the current
 * device after this one (0 restores the default, ~0.1 s of polling; a call
 * captured into a graph keeps the limit it was captured with).  A test hook
 * with no reference counterpart: a limit of 1 makes the waits give up at
 * once, which exercises the give-up path while every kernel still exits
 * normally. */
int32_t l20_pd_set_spin_limit(uint32_t polls);

/* 1 if l20_pd_fp8_e4m3_split_out (or l20_pd_split_out) runs `args` on the
 * current device as the single launch -- one workgroup per (sequence, KV
 * head), the splits folded in LDS, the partial_* workspace neither read nor
 * written, no merge launch --; 2 if its partial stage runs as that kernel's
 * split mode (one workgroup per (split, sequence, KV head), each writing its
 * split's partial) followed by the merge; 0 if as the persistent partial
 * kernel and the merge; -(error code) when the arguments fail
 * l20_pd_fp8_e4m3_check.  Host only.  No reference counterpart: the reference
 * always runs its partial and reduce kernels (l20_paged_decode.cu:692-723).
 * The single launch is taken for G x q_len <= 32 (tree masks included),
 * batch x num_kv_heads <= the CU count and at most 1024 (fp8 caches) or 640
 * (16-bit caches) tokens per sequence within reach of the call; the split
 * mode for 256-, 512- or 1024-token splits whose batch x num_kv_heads x splits
 * triples do not exceed the CUs and, at 512 (1024) tokens, fill at least (more
 * than) half of them. */
int32_t l20_pd_single_launch(const l20_pd_fp8_args *args);

/* Sets every work-queue counter of the current device to `value` (after a
 * device synchronize), as a launch that gave up mid-way or shared a slot with
 * another leaves it.  A test hook with no reference counterpart: with a value
 * that no clean launch produces (e.g. a low half of 2^30), the next call that
 * claims queue items reports L20_PD_DEVERR_QUEUE_SHARED, and
 * l20_pd_device_errors(1) zeroes the counters again. */
int32_t l20_pd_set_queue_counters(uint64_t value);

/* Allocation-free variant of l20_pd_fp8_e4m3_split_out (no counterpart in the
 * reference: for callers that cannot allocate device memory, such as code
 * under HIP graph capture, tight serving loops or harnesses that forbid
 * hipMalloc).  Same arguments and kernels, but the partial_* fields of `args`
 * are ignored: the fp32 split partials go to a 64 MiB array the library holds
 * on each device for the life of the process (its address is looked up once
 * per device, on the first call with that device current).  Calls needing more
 * than 64 MiB of partials (batch*q_len*num_q_heads*ceil(max_seq_len/split_size)
 * *(head_dim+2)*4 bytes) return L20_PD_EINVAL.  The caller passes the inputs,
 * output and (optionally) lse; nothing is allocated.  Every call on a device
 * shares that device's array, so calls that overlap on one device (different
 * streams, or host threads) race and must be serialised by the caller. */
int32_t l20_pd_fp8_e4m3_split_out_noalloc(const l20_pd_fp8_args *args, void *stream);

/* The fp16/bf16-KV sibling: the same two kernels over 16-bit caches
 * (kv_dtype L20_PD_KV_FP16 or L20_PD_KV_BF16, query of the same type; the
 * scalar/per-head scales still multiply K and V, 1.0 reproduces the
 * reference).  With page_indptr set it is the CSR variant. */
int32_t l20_pd_split_out(const l20_pd_fp8_args *args, void *stream);

/* The two stages of l20_pd_fp8_e4m3_split_out, enqueued separately (same
 * arguments, same validation): the split-KV partial kernel
 * (<- paged_decode_fp8_e4m3_partial_kernel, l20_paged_decode.cu:291-422,
 * launched at :692-712) and the LSE merge kernel (<- paged_decode_merge_kernel,
 * l20_paged_decode.cu:424-463, launched at :713-723).  split_out is exactly
 * partial followed by merge; the merge is a no-op when ceil(max_seq_len /
 * split_size) <= 1. */
int32_t l20_pd_fp8_e4m3_partial(const l20_pd_fp8_args *args, void *stream);
int32_t l20_pd_fp8_e4m3_merge(const l20_pd_fp8_args *args, void *stream);

/* Split size the library picks for a call shape when the caller has no
 * preference: a power of two in [64, 1024] -- 1024 above 32768 tokens, else
 * 512, halved while a max_seq_len sequence would have fewer than ~8 splits,
 * then doubled while that lets batch x splits items fit one round of the
 * persistent grid (cu_count x 8 waves / waves per workgroup).
 * (The reference hook passes a fixed 512, install_l20_fp8_paged_decode.py.) */
int32_t l20_pd_default_split_size(int32_t batch, int32_t num_kv_heads,
                                  int32_t max_seq_len, int32_t cu_count);

/* Bulk e4m3fn dequantisation on the GPU: dst[i] = float(src[i]) * scale.
 * Uses the same conversion instruction as the attention kernel's V path. */
int32_t l20_pd_fp8_e4m3_dequant_f32(const uint8_t *src, float *dst, int64_t n,
                                    float scale, void *stream);

/* Bulk e4m3fn -> bf16 (raw uint16 bits) with the attention kernel's K path. */
int32_t l20_pd_fp8_e4m3_dequant_bf16(const uint8_t *src, uint16_t *dst,
                                     int64_t n, void *stream);

/* HBM calibration (no reference counterpart; measurement support).
 * stream_read reads `bytes` once: workgroup i of `blocks` (256 threads)
 * reads the i-th contiguous chunk of ceil(bytes / blocks) bytes, rounded up
 * to 4 KiB, with 16-byte buffer loads (sink: int32 [blocks], practically
 * never written); stream_copy copies `bytes` from src to dst.  Used to measure the
 * device's read ceiling and to scale FETCH_SIZE / WRITE_SIZE counters. */
int32_t l20_pd_stream_read(const void *src, int64_t bytes, int32_t *sink,
                           int32_t blocks, void *stream);
int32_t l20_pd_stream_copy(const void *src, void *dst, int64_t bytes,
                           int32_t blocks, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* L20_PAGED_DECODE_H_ */
