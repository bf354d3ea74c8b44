// Draft-suffix step of hybrid tree attention for MI355X (gfx950): each draft
// row's attention over the contiguous draft keys it may see (the ancestor
// mask), merged with its attention over the paged prefix, in one launch.
//
//  tree_suffix_merge<T, PO, D>   one wave per (sequence, draft row, query head),
//    four waves per workgroup.  Lane l holds dims [l E, l E + E) of the row
//    (E = D / 64).  The wave starts from the prefix state (m = its LSE in log2
//    units, l = 1, acc = its normalised output), reads row i of the ancestor
//    mask with one byte per lane and a ballot, then takes the visible drafts
//    eight at a time: all K and V loads of a batch are issued before any
//    arithmetic, each score is a wave sum of the lanes' partial dots
//    (xor shuffles), and the online softmax folds the batch into (m, l, acc)
//    in fp32.  The work is a few KB per row, so the kernel is latency-bound and
//    a 16-row MFMA tile would sit mostly empty (draft x group rows of one KV
//    head are rarely a multiple of 16, and each row has its own mask).
//
// Reference semantics (paths relative to the reference repo root):
//   src/l20_stack/ops/triton_tree_attention.py:436-510 (_tree_suffix_summary_kernel),
//   :513-545 (_tree_summary_merge_kernel), launched at :1152-1197.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "l20_tree_verify.h"

// Error reporting shared with the decode entry points (l20_pd_last_error).
namespace l20pd_host {
int32_t set_error(int32_t code, const char *msg);
void clear_error();
}  // namespace l20pd_host

namespace l20tv {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBatchKeys = 8;  // draft keys whose loads are in flight together

struct Params {
  const void *q;
  int64_t q_sb, q_ss, q_sh;
  const void *k;
  int64_t k_sb, k_ss, k_sh;
  const void *v;
  int64_t v_sb, v_ss, v_sh;
  const uint8_t *mask;
  int64_t m_sr, m_sc;
  const void *po;
  int64_t po_sb, po_ss, po_sh;
  const float *pl;
  int64_t pl_sb, pl_ss, pl_sh;
  void *out;
  int64_t o_sb, o_ss, o_sh;
  float scale_log2;
  int batch, draft, hq, group;
  int64_t rows;  // batch * draft * hq
};

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <typename T, typename PO, int D>
__global__ __launch_bounds__(256) void tree_suffix_merge(Params p) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // whole waves
  const int h = (int)(row % p.hq);
  const int i = (int)((row / p.hq) % p.draft);
  const int b = (int)(row / ((int64_t)p.hq * p.draft));
  const int kvh = h / p.group;
  const int d0 = lane * E;

  const T *qrow = static_cast<const T *>(p.q) + b * p.q_sb + i * p.q_ss + h * p.q_sh + d0;
  float q[E];
#pragma unroll
  for (int e = 0; e < E; ++e) q[e] = to_f32(qrow[e]) * p.scale_log2;

  // Visible drafts: bit j of the ballot = mask[i][j] != 0.
  const bool vis = lane < p.draft && p.mask[i * p.m_sr + lane * p.m_sc] != 0;
  uint64_t bits = __ballot(vis);

  // Prefix state in log2 units; an empty prefix contributes nothing.
  const float lse = p.pl[b * p.pl_sb + i * p.pl_ss + h * p.pl_sh];
  float m = -INFINITY, l = 0.f, acc[E];
  if (lse > -INFINITY) {
    const PO *prow = static_cast<const PO *>(p.po) + b * p.po_sb + i * p.po_ss + h * p.po_sh + d0;
    m = lse * kLog2e;
    l = 1.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = to_f32(prow[e]);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.f;
  }

  const T *kbase = static_cast<const T *>(p.k) + b * p.k_sb + kvh * p.k_sh + d0;
  const T *vbase = static_cast<const T *>(p.v) + b * p.v_sb + kvh * p.v_sh + d0;
  while (bits) {  // wave-uniform
    int idx[kBatchKeys];
    int n = 0;
#pragma unroll
    for (int t = 0; t < kBatchKeys; ++t) {
      idx[t] = bits ? __builtin_ctzll(bits) : 0;
      if (bits) {
        bits &= bits - 1;
        ++n;
      }
    }
    T kr[kBatchKeys][E], vr[kBatchKeys][E];
#pragma unroll
    for (int t = 0; t < kBatchKeys; ++t)
      if (t < n) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          kr[t][e] = kbase[idx[t] * p.k_ss + e];
          vr[t][e] = vbase[idx[t] * p.v_ss + e];
        }
      }
    float s[kBatchKeys];
    float mb = m;
#pragma unroll
    for (int t = 0; t < kBatchKeys; ++t) {
      s[t] = -INFINITY;
      if (t < n) {
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) part += q[e] * to_f32(kr[t][e]);
        s[t] = wave_sum(part);
        mb = fmaxf(mb, s[t]);
      }
    }
    // mb is finite: at least one key of the batch is visible.
    const float c = exp2f(m - mb);  // 0 when m = -inf
    l *= c;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] *= c;
#pragma unroll
    for (int t = 0; t < kBatchKeys; ++t)
      if (t < n) {
        const float pr = exp2f(s[t] - mb);
        l += pr;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] += pr * to_f32(vr[t][e]);
      }
    m = mb;
  }

  const float inv = l > 0.f ? 1.f / l : 0.f;
  T *orow = static_cast<T *>(p.out) + b * p.o_sb + i * p.o_ss + h * p.o_sh + d0;
#pragma unroll
  for (int e = 0; e < E; ++e) orow[e] = (T)(acc[e] * inv);
}

}  // namespace l20tv

namespace {

using l20pd_host::set_error;

int32_t check(const l20_pd_tree_suffix_args *a) {
  if (!a) return set_error(L20_PD_EINVAL, "null arguments");
  if (a->query_dtype != L20_PD_BF16 && a->query_dtype != L20_PD_FP16)
    return set_error(L20_PD_EINVAL, "query must be bf16 or fp16");
  if (a->prefix_dtype != a->query_dtype && a->prefix_dtype != L20_PD_FP32)
    return set_error(L20_PD_EINVAL, "prefix output must have the query dtype or fp32");
  if (a->head_dim != 64 && a->head_dim != 128) return set_error(L20_PD_EINVAL, "head_dim must be 64 or 128");
  if (a->draft_length < 1 || a->draft_length > 64)
    return set_error(L20_PD_EINVAL, "paged suffix path supports draft_length in [1, 64]");
  if (a->batch < 0 || a->num_q_heads < 1 || a->num_kv_heads < 1 || a->num_q_heads % a->num_kv_heads)
    return set_error(L20_PD_EINVAL, "requires an integral GQA ratio");
  if (a->batch > 0 && (!a->query || !a->suffix_key || !a->suffix_value || !a->ancestor_mask || !a->prefix_output ||
                       !a->prefix_lse || !a->output))
    return set_error(L20_PD_EINVAL, "null tensor pointer");
  if (!(a->softmax_scale > 0.f) || !isfinite(a->softmax_scale))
    return set_error(L20_PD_EINVAL, "softmax_scale must be positive and finite");
  return L20_PD_OK;
}

l20tv::Params params(const l20_pd_tree_suffix_args &a) {
  l20tv::Params p;
  p.q = a.query;
  p.q_sb = a.q_stride_batch;
  p.q_ss = a.q_stride_draft;
  p.q_sh = a.q_stride_head;
  p.k = a.suffix_key;
  p.k_sb = a.sk_stride_batch;
  p.k_ss = a.sk_stride_draft;
  p.k_sh = a.sk_stride_head;
  p.v = a.suffix_value;
  p.v_sb = a.sv_stride_batch;
  p.v_ss = a.sv_stride_draft;
  p.v_sh = a.sv_stride_head;
  p.mask = a.ancestor_mask;
  p.m_sr = a.mask_stride_row;
  p.m_sc = a.mask_stride_col;
  p.po = a.prefix_output;
  p.po_sb = a.po_stride_batch;
  p.po_ss = a.po_stride_draft;
  p.po_sh = a.po_stride_head;
  p.pl = a.prefix_lse;
  p.pl_sb = a.pl_stride_batch;
  p.pl_ss = a.pl_stride_draft;
  p.pl_sh = a.pl_stride_head;
  p.out = a.output;
  p.o_sb = a.o_stride_batch;
  p.o_ss = a.o_stride_draft;
  p.o_sh = a.o_stride_head;
  p.scale_log2 = a.softmax_scale * l20tv::kLog2e;
  p.batch = a.batch;
  p.draft = a.draft_length;
  p.hq = a.num_q_heads;
  p.group = a.num_q_heads / a.num_kv_heads;
  p.rows = (int64_t)a.batch * a.draft_length * a.num_q_heads;
  return p;
}

template <typename T, typename PO>
void launch_dim(const l20tv::Params &p, int head_dim, hipStream_t s) {
  const dim3 grid((unsigned)((p.rows + 3) / 4));
  if (head_dim == 128)
    hipLaunchKernelGGL((l20tv::tree_suffix_merge<T, PO, 128>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((l20tv::tree_suffix_merge<T, PO, 64>), grid, dim3(256), 0, s, p);
}

}  // namespace

extern "C" {

int32_t l20_pd_tree_suffix_check(const l20_pd_tree_suffix_args *a) {
  l20pd_host::clear_error();
  return check(a);
}

int32_t l20_pd_tree_suffix_merge(const l20_pd_tree_suffix_args *a, void *stream) {
  l20pd_host::clear_error();
  const int32_t rc = check(a);
  if (rc != L20_PD_OK) return rc;
  const l20tv::Params p = params(*a);
  if (p.rows == 0) return L20_PD_OK;
  if ((p.rows + 3) / 4 >= ((int64_t)1 << 31)) return set_error(L20_PD_EINVAL, "too many rows");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool f32 = a->prefix_dtype == L20_PD_FP32;
  if (a->query_dtype == L20_PD_BF16) {
    if (f32) launch_dim<__bf16, float>(p, a->head_dim, s);
    else launch_dim<__bf16, __bf16>(p, a->head_dim, s);
  } else {
    if (f32) launch_dim<_Float16, float>(p, a->head_dim, s);
    else launch_dim<_Float16, _Float16>(p, a->head_dim, s);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[256];
    snprintf(msg, sizeof(msg), "HIP launch failed: %s", hipGetErrorString(e));
    return set_error(L20_PD_ELAUNCH, msg);
  }
  return L20_PD_OK;
}

}  // extern "C"
