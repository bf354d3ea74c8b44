// Paged FP8 (OCP e4m3fn) KV-cache decode attention for MI355X (gfx950).
//
// Two kernels per call, both enqueued on the caller's stream:
//
//  pd_fp8_partial<QT, KT, D, NQT, TREE, NB>  persistent: CUs x occupancy workgroups, one
//    wave per KV head (W waves, W the largest divisor of Hkv up to 8).
//    A work item is one (sequence, split) pair; every wave of the workgroup
//    computes attention for ALL query rows of its KV head (GQA group x
//    q_len, padded to 16 * NQT MFMA columns), so each K/V page is read from
//    HBM exactly once.  Each wave streams 32-token blocks through NB (1 or 2)
//    register buffers without draining between items (the next item's page
//    ids, query and first blocks load while the current one finishes).
//    Per block and lane:
//      K: 2 tiles x D/64 x 16 B loads (token = lane%16, 64-byte half-rows),
//         fp8 -> bf16/f16 conversion (exact), S^T = K . Q^T on
//         v_mfma_f32_16x16x32_{bf16,f16}: rows = tokens, columns = query rows.
//      softmax: each lane holds 8 scores of one query column; the block max is
//         reduced across the four 16-lane groups; exp2 with the K scale, the
//         softmax scale and log2(e) folded into one multiplier.
//      V: 8 tokens x D/16 contiguous bytes per lane; a byte permute and the
//         fp8 -> f16 conversion pack token pairs, which transposes V for the
//         MFMA A operand in registers (no LDS pass).  O^T += V^T . P^T with P
//         in f16.
//    A sequence with a single split writes the final output and LSE;
//    otherwise the fp32 partial (O / l, m, l) goes to the caller's workspace.
//
//  pd_merge<QT, D, WPP, PK, SPEC>   WPP waves per (query row, q head), WPP from the split
//    count; PK the partial element (0 fp32, 1 fp16, 2 bf16).  pd_merge_narrow<QT, D, PK>
//    for at most eight splits and many pairs.
//    LSE merge of a row's splits: M = max m_s, w_s = 2^(m_s - M) l_s,
//    out = sum w_s o_s / sum w_s, lse = ln2 (M + log2 sum w_s).
//
// Reference semantics (paths relative to the reference repo root):
//   integrations/vllm/cuda/l20_paged_decode.cu:291-422 (partial),
//   :424-463 (merge), :651-725 (host launcher and argument checks);
//   scripts/smoke_cuda_paged_fp8_decode_op.py:22-41 (dequantise-then-attend).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "l20_paged_decode.h"

namespace l20pd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int kPage = 16;
constexpr int kMaxWaves = 8;       // waves per partial workgroup (one per KV head)
constexpr int kMaxCompactBatch = 4096;  // sequences whose work list fits in LDS
// Hand-off leads, in blocks before a unit's end, for a stream of NB blocks in
// flight: the successor is needed NB + 1 blocks before the end (its first
// block is the refill after the next step), published 3 blocks earlier and
// claimed 3 blocks before that.
constexpr int need_lead(int nb) { return nb + 1; }
constexpr int publish_lead(int nb) { return nb + 4; }
constexpr int claim_lead(int nb) { return nb + 7; }
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer resource: dword 3 (format bits)
// Cache policy of the K/V stream loads: non-temporal (the CPol NT bit).  Every
// K/V byte is read once per call; on MI355X a streaming read with NT reaches
// ~7.1 TB/s against ~6.35 TB/s with the default policy.
constexpr int kStreamPolicy = 2;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleLog2 = 8.0f;  // lazy online-softmax rescale threshold (log2 units)

struct PartialParams {
  const void *q;
  int64_t q_srow, q_shead;
  const uint8_t *k;
  int64_t k_spage;
  int k_stok32, k_shead32, k_extent;
  const uint8_t *v;
  int64_t v_spage;
  int v_stok32, v_shead32, v_extent;
  const int32_t *bt;
  int64_t bt_srow;
  const int32_t *seq_lens;
  int64_t num_pages;
  void *po;
  int64_t po_srow, po_shead, po_ssplit;
  float *pm;
  int64_t pm_srow, pm_shead, pm_ssplit;
  float *pl;
  int64_t pl_srow, pl_shead, pl_ssplit;
  void *out;
  int64_t o_srow, o_shead;
  float *lse;
  int64_t lse_srow, lse_shead;
  float k_scale, v_scale;
  const float *k_scale_ph;
  const float *v_scale_ph;
  float qk_scale_log2;  // softmax_scale * log2(e)
  int q_len, num_q_heads, num_kv_heads, group, split_size, num_splits;
  int po_kind;  // partial o/l element: 0 fp32, 1 fp16, 2 bf16
  int l_cap;  // min(num_splits * split_size, block-table pages * page_size): tokens past it are never touched
  int batch;
  int bt_pages;  // block-table row length
  int compact;   // queue items numbered through an LDS prefix
  const int32_t *indptr;  // CSR page list: sequence b's pages are bt[indptr[b] .. indptr[b + 1])
  const int32_t *tree;    // ancestor words [b * tree_sb + i] (bit j: row i sees draft key j), or NULL
  int64_t tree_sb;
  int queue_slot;  // the launch's work-queue counters (g_pd_queue row)
  // Two items per workgroup (kernels that support it): waves [0, W) and
  // [W, 2W) are two independent groups, virtual workgroups blockIdx.x and
  // gridDim.x + blockIdx.x of the schedule.
  int paired;
  // Polls before a hand-off wait gives up: kSpinLimit unless lowered through
  // l20_pd_set_spin_limit (tests force the give-up path with it).
  unsigned int spin_cap;
  // Host launch number, mixed into the launch's work-queue tag.
  unsigned int launch_tag;
  // 16-token tiles per page-list entry (pages of 16 * page_mult tokens, their
  // tokens contiguous): tile T of a sequence is sub-page T % page_mult of
  // entry T / page_mult, virtual page entry * page_mult + T % page_mult of a
  // cache seen as 16-token pages (num_pages and the page stride are given in
  // those).
  int page_mult;
  // ceil(2^32 / page_mult) (page_mult > 1): T / page_mult = umulhi(T, magic),
  // exact for T < 2^32 / page_mult (the host bounds max_seq_len for it).
  unsigned int page_magic;
  // pd_fp8_fused only: 0 = one workgroup per (sequence, KV head) covers the
  // whole sequence; otherwise the split size, one workgroup per (split,
  // sequence, KV head) writing the split's partial for the merge.
  int fused_split;
};

// ---------------------------------------------------------------------------
// Element helpers
// ---------------------------------------------------------------------------
template <typename QT> struct MfmaTypes;
template <> struct MfmaTypes<__bf16> { typedef bf16x8 vec8; };
template <> struct MfmaTypes<_Float16> { typedef f16x8 vec8; };

// Eight fp8 codes (two dwords) -> eight bf16 / f16 MFMA operand elements,
// exact (every e4m3fn and every e5m2 value is representable in both).
// gfx950 v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8} (fp8 = OCP e4m3, bf8 = OCP
// e5m2) with scale 1.0, word_sel picking bytes 0-1 or 2-3.  The pairs are
// moved as whole 32-bit words: per-lane extraction of these conversions'
// results is miscompiled by the ROCm 7.2 LLVM.
template <bool E5M2> __device__ __forceinline__ int cvt_pk_bf16(int w, bool hi) {
  if constexpr (E5M2)
    return hi ? __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true))
              : __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false));
  else
    return hi ? __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true))
              : __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
template <bool E5M2> __device__ __forceinline__ int cvt_pk_f16(int w, bool hi) {
  if constexpr (E5M2)
    return hi ? __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, true))
              : __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, false));
  else
    return hi ? __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true))
              : __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}
template <typename V8, bool E5M2> __device__ __forceinline__ V8 fp8x8_to(int w0, int w1);
template <> __device__ __forceinline__ bf16x8 fp8x8_to<bf16x8, false>(int w0, int w1) {
  const i32x4 r = {cvt_pk_bf16<false>(w0, false), cvt_pk_bf16<false>(w0, true), cvt_pk_bf16<false>(w1, false),
                   cvt_pk_bf16<false>(w1, true)};
  return __builtin_bit_cast(bf16x8, r);
}
template <> __device__ __forceinline__ bf16x8 fp8x8_to<bf16x8, true>(int w0, int w1) {
  const i32x4 r = {cvt_pk_bf16<true>(w0, false), cvt_pk_bf16<true>(w0, true), cvt_pk_bf16<true>(w1, false),
                   cvt_pk_bf16<true>(w1, true)};
  return __builtin_bit_cast(bf16x8, r);
}
template <> __device__ __forceinline__ f16x8 fp8x8_to<f16x8, false>(int w0, int w1) {
  const i32x4 r = {cvt_pk_f16<false>(w0, false), cvt_pk_f16<false>(w0, true), cvt_pk_f16<false>(w1, false),
                   cvt_pk_f16<false>(w1, true)};
  return __builtin_bit_cast(f16x8, r);
}
template <> __device__ __forceinline__ f16x8 fp8x8_to<f16x8, true>(int w0, int w1) {
  const i32x4 r = {cvt_pk_f16<true>(w0, false), cvt_pk_f16<true>(w0, true), cvt_pk_f16<true>(w1, false),
                   cvt_pk_f16<true>(w1, true)};
  return __builtin_bit_cast(f16x8, r);
}

__device__ __forceinline__ f32x4 mfma16(const bf16x8 &a, const bf16x8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(const f16x8 &a, const f16x8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Empty asm statements that take a value in VGPRs: the loads producing it
// complete at this point instead of at its first use.
template <typename V8, int A, int B> __device__ __forceinline__ void pin_operands(V8 (&x)[A][B]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) {
      i32x4 w = __builtin_bit_cast(i32x4, x[a][b]);
      asm volatile("" : "+v"(w));
      x[a][b] = __builtin_bit_cast(V8, w);
    }
}
template <int N> __device__ __forceinline__ void pin_words(int (&x)[N]) {
#pragma unroll
  for (int a = 0; a < N; ++a) asm volatile("" : "+v"(x[a]));
}

// Byte pair (sel=0: bytes 0,1; sel=1: bytes 2,3) of a dword -> two f32.
template <bool E5M2> __device__ __forceinline__ f32x2 fp8x2_f32(int w, bool hi) {
  if constexpr (E5M2)
    return hi ? __builtin_amdgcn_cvt_pk_f32_bf8(w, true) : __builtin_amdgcn_cvt_pk_f32_bf8(w, false);
  else
    return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true) : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
}

template <typename QT> __device__ __forceinline__ QT from_f32(float x);
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }

// Reductions over lanes l, l^16, l^32 and l^48 done in VGPRs, not through
// LDS: with both operands the same register, v_permlane16_swap returns per
// lane the values of the even and the odd 16-lane row of its row pair, and
// v_permlane32_swap those of the two 32-lane halves, so combining the two
// results gives every lane the pair (l, l^16), then (l, l^32).  Both lanes of
// a pair combine the same two operands (fmax and + commute exactly), so all
// four lanes end with the same bits.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
template <int W> __device__ __forceinline__ u32x2_t swap_rows(float x) {
  const unsigned int b = __builtin_bit_cast(unsigned int, x);
  if constexpr (W == 16) return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_permlane16_swap(b, b, false, false));
  else return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_permlane32_swap(b, b, false, false));
}
// The element is taken by value: hipcc lowers __builtin_bit_cast of an
// ext_vector element expression (v[1]) to a load of element 0.
__device__ __forceinline__ float word_f(unsigned int w) { return __builtin_bit_cast(float, w); }
__device__ __forceinline__ float lo_f(u32x2_t v) { return word_f(v[0]); }
__device__ __forceinline__ float hi_f(u32x2_t v) { return word_f(v[1]); }
__device__ __forceinline__ float wave_max_xor16_32(float x) {
  u32x2_t r = swap_rows<16>(x);
  x = fmaxf(lo_f(r), hi_f(r));
  r = swap_rows<32>(x);
  return fmaxf(lo_f(r), hi_f(r));
}
__device__ __forceinline__ float wave_sum_xor16_32(float x) {
  u32x2_t r = swap_rows<16>(x);
  x = lo_f(r) + hi_f(r);
  r = swap_rows<32>(x);
  return lo_f(r) + hi_f(r);
}

// Raw fp8 bytes of one 32-token block (two 16-token pages) held by one lane.
template <int D> struct BlockRaw;
template <> struct BlockRaw<128> {
  i32x4 k[2][2];  // [tile][half-row chunk]: 16 B at d = 64*c + 16*(lane/16)
  i32x2 v[8];     // [token slot]: 8 B at d = 8*(lane%16)
};
template <> struct BlockRaw<64> {
  i32x4 k[2][1];
  int v[8];       // 4 B at d = 4*(lane%16)
};

// Raw fp16/bf16 elements of one 16-token block (one page) held by one lane.
template <int D> struct BlockRaw16;
template <> struct BlockRaw16<128> {
  i32x4 k[4];  // [k slice]: 8 elements at d = 64*(s/2) + 16*(lane/16) + 8*(s%2)
  i32x4 v[4];  // [token slot]: 8 elements at d = 8*(lane%16)
};
template <> struct BlockRaw16<64> {
  i32x4 k[2];
  i32x2 v[4];  // 4 elements at d = 4*(lane%16)
};
// KT = 0: e4m3fn codes, 32-token blocks; KT = 2: e5m2 codes, the same; KT =
// 1: 16-bit elements of the MFMA type, 16-token blocks (the same bytes per
// register buffer).
template <int KT, int D> struct KvBlock { typedef BlockRaw<D> type; };
template <int D> struct KvBlock<1, D> { typedef BlockRaw16<D> type; };

// ---------------------------------------------------------------------------
// Partial kernel
// ---------------------------------------------------------------------------
// Two fp32 -> packed 16-bit words (bf16 or f16, round to nearest even).
// p - (float)h, h the low (HI = 0) or high f16 half of w, in one VOP3P mix
// instruction: the f16 operand widens exactly and the f32 result is rounded
// once (p - h is exact anyway).  hipcc forms no mix instruction from
// fmaf((float)h, -1, p), hence the inline assembly.
template <int HI> __device__ __forceinline__ float sub_half(int w, float p) {
  float r;
  if constexpr (HI) asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(p));
  else asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(p));
  return r;
}

template <typename QT> __device__ __forceinline__ int pack2(float a, float b);
template <> __device__ __forceinline__ int pack2<__bf16>(float a, float b) {
  return __builtin_bit_cast(int, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <> __device__ __forceinline__ int pack2<_Float16>(float a, float b) {
  return __builtin_bit_cast(int, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// Wave-uniform reads of the call's read-only inputs (lengths, CSR offsets,
// per-head scales) go through the constant address space, so they are scalar
// loads counted by lgkmcnt: a vector load would be counted by vmcnt, and
// waiting for it would also wait for every K/V block in flight.
template <typename T> __device__ __forceinline__ T uniform_ld(const T *a, int64_t i) {
  typedef const __attribute__((address_space(4))) T *ConstPtr;
  return ((ConstPtr)a)[i];  // an address-space cast: C-style, as C++ casts do not convert address spaces
}

// Clamped length of sequence b (tokens past l_cap are never touched).
__device__ __forceinline__ int clamped_len(const PartialParams &p, int b) {
  return max(0, min(uniform_ld(p.seq_lens, b), p.l_cap));
}

// Inclusive scan of one value per thread over the workgroup (<= 512 threads).
__device__ __forceinline__ int block_inclusive_scan(int v, int *s_wave) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off);
    if (lane >= off) v += t;
  }
  if (lane == 63) s_wave[wave] = v;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += s_wave[w];
  __syncthreads();
  return v + base;
}

__device__ __forceinline__ int lds_uniform(const int *a, int i) { return __builtin_amdgcn_readfirstlane(a[i]); }

// Relaxed workgroup-scope accesses to the LDS words that waves poll and
// publish.  Atomic rather than volatile: the compiler keeps these as LDS
// instructions (counted by lgkmcnt), whereas volatile LDS accesses become FLAT
// instructions, which also count in vmcnt and so wait for every K/V load in
// flight.
__device__ __forceinline__ int lds_poll(int *a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void lds_put(int *a, int v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Release store / acquire load at workgroup scope: the publication of a
// word that other waves poll, and the poll that reads it (every LDS access
// of the publisher before the store is visible to a wave whose acquire load
// returns the stored value).
#ifndef L20_PD_LDS_ORDER
#define L20_PD_LDS_ORDER 1
#endif
__device__ __forceinline__ void lds_publish(int *a, int v) {
#if L20_PD_LDS_ORDER
  __hip_atomic_store(a, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
#else
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#endif
}
__device__ __forceinline__ int lds_acquire(int *a) {
#if L20_PD_LDS_ORDER
  return __hip_atomic_load(a, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
#else
  const int v = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return v;
#endif
}
#if L20_PD_LDS_ORDER
#define L20_PD_LDS_REL __ATOMIC_RELEASE
#else
#define L20_PD_LDS_REL __ATOMIC_RELAXED
#endif

__device__ __forceinline__ int splits_of_len(int len, int split) { return len > 0 ? (len + split - 1) / split : 1; }
// Work queues of the persistent partial kernel, one per launch slot (one
// 64-byte line each; its first 8 bytes are the counter).  Zero at load.  A
// launch whose grid covers every split-major slot claims nothing.  Otherwise
// every workgroup claims until a claim fails (returns >= Q, the queue length),
// so exactly gridDim.x claims fail and the one that returns Q + gridDim.x - 1
// is the last atomic on the counter in this launch: its workgroup resets the
// counter, and every launch starts from zero without a memset (a captured
// graph replays correctly).  Claims on one line are served one at a time
// (~11 ns each on MI355X), which is why nothing else (such as a count of
// finished workgroups) shares it.
//
// A claim adds 1 + (tag << 32), tag being the launch's own 32-bit tag (a
// host launch number mixed with the address of the launch's dispatch
// packet, so two replays of one graph differ too): after k claims of one
// launch the counter holds k in its low half and k * tag in its high half.
// A claim that returns any other pair came after a claim of another launch
// (two launches overlapping on one slot) or after one that gave up mid-way:
// the workgroup records L20_PD_DEVERR_QUEUE_SHARED and stops claiming.
constexpr int kQueueSlots = 64;
__device__ __align__(64) unsigned long long g_pd_queue[kQueueSlots][8];
// Hand-off waits give up after this many polls (s_sleep 1 each, ~0.1 s in
// all; a wait that the protocol satisfies ends within microseconds).  A wave
// that gives up ORs an L20_PD_DEVERR_* code into g_pd_error[slot], takes no
// further item and exits normally, so a hand-off bug shows up as an error
// (l20_pd_device_errors) instead of a hung GPU.
constexpr unsigned int kSpinLimit = 1u << 22;
__device__ unsigned int g_pd_error[kQueueSlots];

// ---------------------------------------------------------------------------
// Per-unit math of the partial kernel
// ---------------------------------------------------------------------------
// A unit is one wave's scan of one KV head over a token range of one
// sequence.  Lane layout: n16 = lane % 16 is query column 16*qt + n16 of the
// MFMA tile (G x q_len query rows, padded to 16 * NQT), j = lane / 16.
// Blocks hold 32 fp8 tokens (two 16-token pages: tiles 2*blk, 2*blk + 1 of
// the unit's page-id window) or 16 tokens of a 16-bit cache (tile blk).
template <typename QT, int KT, int D, int NQT, bool TREE, bool KLINES>
struct KvUnit {
  typedef typename MfmaTypes<QT>::vec8 qvec8;
  typedef typename KvBlock<KT, D>::type Block;
  // Softmax probabilities: f16 for fp8 caches (V converted to f16), the
  // cache's own type for 16-bit caches.
  typedef typename std::conditional<KT != 1, _Float16, QT>::type PT;
  typedef typename MfmaTypes<PT>::vec8 pvec8;
  static constexpr int kTok = KT != 1 ? 32 : 16;  // tokens per block
  // P is rounded to the MFMA operand type, 11 significant bits (f16) or 8
  // (bf16), while the softmax denominator sums it unrounded.  Equal scores
  // round alike, so the error does not average out: with every other key at
  // p = 2^-0.1 and V = +-448 it reaches ~0.1 absolute.  Split P = hi + lo
  // (hi = rnd(p), lo = rnd(p - hi)) and accumulate both products: ~22 (f16) or
  // ~16 (bf16) bits.
  static constexpr bool kSplitP = true;
  static constexpr int NCH = D / 64;  // 64-byte K chunks per token row
  static constexpr int NS = 2 * NCH;  // 32-wide k slices of the QK product
  static constexpr int NT = D / 16;   // 16-row d tiles of the PV product
  static constexpr int DPL = D / 4;   // contiguous output dims per lane
  // KLINES (fp8 K at head_dim 128; not for two query tiles with two blocks
  // in flight, which would spill more): K arrives in whole
  // 128-byte lines (lane l: token 8c + l/8 of page T, bytes 16 (l % 8)) and
  // goes through the wave's own LDS rows into the MFMA layout (lane (n16, j):
  // token n16, bytes 16 j + 64 c).  Loading the MFMA layout straight from
  // memory takes half of 16 lines per instruction; in load-only kernels over
  // the config-3 pages and schedule that streamed at 4.7 TB/s against 5.6 for
  // whole lines.  In the full kernels the pass gains 1.6 us at config 4 (85.4
  // vs 87.1 us, same box) and nothing at config 5, both one block in flight;
  // in the two-block kernel of config 3 it gains 1.4 us once that kernel's
  // loads are issued in the same order on every path (it cost 1.1 us while the
  // compiler drained the stream before every other block).  Rows are padded
  // to 144 bytes so that the 16 rows of a read fall in distinct banks.
  static constexpr bool kKLines = KLINES;
  static constexpr int kKxRow = 144;                  // LDS bytes per token row
  static constexpr int kKxBytes = 2 * 16 * kKxRow;    // two pages per block

  // online-softmax state: O^T tiles, running max (log2 units) and sum per column
  f32x4 acc[NQT][NT];
  float m_run[NQT], l_run[NQT];

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      m_run[qt] = -INFINITY;
      l_run[qt] = 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // Raw buffer loads through a per-page resource: the page base lives in
  // SGPRs, one 32-bit lane offset serves every K (V) load of the page and the
  // hardware range check (the page's byte extent) returns zeros for anything
  // outside it.  Loads are unconditional -- an invalid page id, or none, reads
  // zeros through a zero-extent resource -- and compute_block masks every
  // token outside the unit or on an invalid page and zeroes its V.  Lane offsets inside a page fit in 32 bits (checked on the
  // host).  parts: 1 = the K loads, 2 = the V loads, 3 = both.
  static constexpr int kPagesPerBlock = KT == 1 ? 1 : 2;
  // Page ids of block blk of a unit (lane t of pid holds tile t's id, -1 for
  // none), wave-uniform.
  static __device__ __forceinline__ void block_pages(int pid, int blk, int (&pg)[2]) {
#pragma unroll
    for (int T = 0; T < 2; ++T) pg[T] = T < kPagesPerBlock ? __builtin_amdgcn_readlane(pid, kPagesPerBlock * blk + T) : -1;
  }
  static __device__ __forceinline__ void load_block(const PartialParams &p, Block &r, int pid, int kvh, int blk,
                                                    int parts, int n16, int j) {
    int pg[2];
    block_pages(pid, blk, pg);
    load_pages(p, r, pg, kvh, parts, n16, j);
  }
  // The loads of one block from its pages: straight-line code, no branch
  // around any load, K of every page before V of every page (a refill issued
  // in two parts keeps the same order).  A page id below 0 (none, or an
  // invalid one) gets a resource of zero extent: its loads return zeros
  // without touching memory, and compute_block masks those tokens.
  static __device__ __forceinline__ void load_pages(const PartialParams &p, Block &r, const int (&pg)[2], int kvh,
                                                    int parts, int n16, int j) {
    if constexpr (KT == 1) {
      // 16-bit elements: one page per block; K slice s at byte 128*(s/2) + 16*(s%2)
      const uint32_t koff = (uint32_t)(n16 * p.k_stok32 + kvh * p.k_shead32 + 32 * j);
      const uint32_t voff = (uint32_t)(4 * j * p.v_stok32 + kvh * p.v_shead32 + 2 * (D / 16) * n16);
      const int page = max(pg[0], 0);
      const bool live = pg[0] >= 0;
      if (parts & 1) {
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(p.k) + (int64_t)page * p.k_spage, (short)0, live ? p.k_extent : 0, kBufferWord3);
#pragma unroll
        for (int s = 0; s < NS; ++s)
          r.k[s] = __builtin_bit_cast(
              i32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff, 128 * (s >> 1) + 16 * (s & 1), kStreamPolicy));
      }
      if (parts & 2) {
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(p.v) + (int64_t)page * p.v_spage, (short)0, live ? p.v_extent : 0, kBufferWord3);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (D == 128)
            r.v[e] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff, e * p.v_stok32, kStreamPolicy));
          else
            r.v[e] = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(vr, voff, e * p.v_stok32, kStreamPolicy));
        }
      }
    } else {
      const int lane = n16 + 16 * j;
      // whole lines (kKLines): token 8c + lane / 8 of the page, 16 bytes at 16 (lane % 8)
      const uint32_t koff = kKLines ? (uint32_t)((lane >> 3) * p.k_stok32 + kvh * p.k_shead32 + 16 * (lane & 7))
                                    : (uint32_t)(n16 * p.k_stok32 + kvh * p.k_shead32 + 16 * j);
      const uint32_t voff = (uint32_t)(4 * j * p.v_stok32 + kvh * p.v_shead32 + (D / 16) * n16);
      if (parts & 1) {
#pragma unroll
        for (int T = 0; T < 2; ++T) {
          const __amdgpu_buffer_rsrc_t kr =
              __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.k) + (int64_t)max(pg[T], 0) * p.k_spage,
                                                (short)0, pg[T] >= 0 ? p.k_extent : 0, kBufferWord3);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            r.k[T][c] = __builtin_bit_cast(
                i32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff, kKLines ? 8 * c * p.k_stok32 : 64 * c,
                                                             kStreamPolicy));
        }
      }
      if (parts & 2) {
#pragma unroll
        for (int T = 0; T < 2; ++T) {
          const __amdgpu_buffer_rsrc_t vr =
              __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.v) + (int64_t)max(pg[T], 0) * p.v_spage,
                                                (short)0, pg[T] >= 0 ? p.v_extent : 0, kBufferWord3);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (D == 128)
              r.v[4 * T + e] = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(vr, voff, e * p.v_stok32, kStreamPolicy));
            else
              r.v[4 * T + e] = (int)__builtin_amdgcn_raw_buffer_load_b32(vr, voff, e * p.v_stok32, kStreamPolicy);
          }
        }
      }
    }
  }

  // Query operand (B of S^T = K . Q^T): column n' = 16*qt + lane%16.
  static __device__ __forceinline__ void load_q(const PartialParams &p, int b, int kvh, qvec8 (&dst)[NQT][NS], int n16,
                                                int j) {
    const int q_len = p.q_len;
    const int mcols = p.group * q_len;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const int col = 16 * qt + n16;
      const int g = col / q_len;
      const int i = col - g * q_len;
      if (col < mcols) {
        const QT *qrow = reinterpret_cast<const QT *>(p.q) + (int64_t)(b * q_len + i) * p.q_srow +
                         (int64_t)(kvh * p.group + g) * p.q_shead;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int d0 = (s >> 1) * 64 + 16 * j + (s & 1) * 8;
          dst[qt][s] = __builtin_bit_cast(qvec8, *reinterpret_cast<const i32x4 *>(qrow + d0));
        }
      } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) dst[qt][s] = __builtin_bit_cast(qvec8, i32x4{0, 0, 0, 0});
      }
    }
  }

  // Tree verification: ancestor words of this lane's query columns over the
  // newest q_len keys (bit j lets the column see key L - q_len + j).  The
  // causal rule (TREE = false) keeps no words: its limit is recomputed per
  // unit, which keeps the tree state out of the causal kernels' registers.
  static __device__ __forceinline__ void load_tree(const PartialParams &p, int b, int (&dst)[TREE ? NQT : 1], int n16) {
    if constexpr (TREE) {
      const int mcols = p.group * p.q_len;
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        const int col = 16 * qt + n16;
        dst[qt] = col < mcols ? p.tree[(int64_t)b * p.tree_sb + (col % p.q_len)] : 0;
      }
    }
  }

  // One block: tokens tok0 .. tok0 + kTok - 1 of the sequence, page ids in
  // lanes kTilesPerBlock*blk (+1) of pid.  Keys at or past uEnd, on an
  // invalid page, or hidden by the mask get score -inf and zero V.  Keys
  // before draft0 are visible to every column; key draft0 + j to draft row i
  // when j <= i (causal: lim is the lane column's last visible key) or when
  // bit j of the row's ancestor word is set (TREE); min_lim is the last key
  // every column sees.  after_scores() runs once r.k has been consumed.
  // Whole-line K (kKLines) -> the MFMA layout through the wave's LDS rows kx.
  // The writes and reads of one wave are ordered by the LDS pipeline, and the
  // previous block's reads of kx precede these writes in program order.
  static __device__ __forceinline__ void k_to_mfma(Block &r, char *kx, int n16, int j) {
    const int lane = n16 + 16 * j;
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        *reinterpret_cast<i32x4 *>(kx + T * 16 * kKxRow + (8 * c + (lane >> 3)) * kKxRow + 16 * (lane & 7)) =
            r.k[T][c];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        r.k[T][c] = *reinterpret_cast<const i32x4 *>(kx + T * 16 * kKxRow + n16 * kKxRow + 16 * j + 64 * c);
  }

  template <typename F>
  __device__ __forceinline__ void compute_block(Block &r, int pid, int blk, int tok0, int uEnd, int draft0,
                                                const int (&lim)[TREE ? 1 : NQT], int min_lim,
                                                const int (&tree)[TREE ? NQT : 1], const qvec8 (&qop)[NQT][NS],
                                                float c_log2, int j, char *kx, F &&after_scores) {
    // Tokens past the unit (the tail of the sequence's last page, or a tile
    // beyond the unit read from page 0) and tokens of an invalid page may hold
    // arbitrary bytes, NaN codes included: zero their V so that p = 0
    // contributes exactly 0.  K needs no fix-up: their scores are replaced by
    // -inf below.  A 16-bit block has one tile; its second-tile slots are
    // empty (score -inf, V zero).
    const bool bad0 = __builtin_amdgcn_readlane(pid, KT != 1 ? 2 * blk : blk) < 0;
    const bool bad1 = KT != 1 ? __builtin_amdgcn_readlane(pid, 2 * blk + 1) < 0 : true;
    if constexpr (KT != 1) {
      if (tok0 + 32 > uEnd || bad0 || bad1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = tok0 + 16 * (e >> 2) + 4 * j + (e & 3);
          if (t >= uEnd || ((e >> 2) ? bad1 : bad0)) {
            if constexpr (D == 128)
              r.v[e] = i32x2{0, 0};
            else
              r.v[e] = 0;
          }
        }
      }
    } else {
      if (tok0 + 16 > uEnd || bad0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (tok0 + 4 * j + e >= uEnd || bad0) {
            if constexpr (D == 128)
              r.v[e] = i32x4{0, 0, 0, 0};
            else
              r.v[e] = i32x2{0, 0};
          }
        }
      }
    }
    if constexpr (kKLines) k_to_mfma(r, kx, (int)(threadIdx.x & 15), j);
    // ---- S^T = K . Q^T ----
    f32x4 sc[NQT][2];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      sc[qt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      sc[qt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (KT != 1) {
#pragma unroll
      for (int T = 0; T < 2; ++T) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const i32x4 raw = r.k[T][s >> 1];
          const qvec8 kop = fp8x8_to<qvec8, KT == 2>(raw[2 * (s & 1)], raw[2 * (s & 1) + 1]);
#pragma unroll
          for (int qt = 0; qt < NQT; ++qt) sc[qt][T] = mfma16(kop, qop[qt][s], sc[qt][T]);
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const qvec8 kop = __builtin_bit_cast(qvec8, r.k[s]);
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) sc[qt][0] = mfma16(kop, qop[qt][s], sc[qt][0]);
      }
    }
    // r.k is consumed: the refill's K loads may overwrite it
    after_scores();
    // ---- online softmax (log2 domain) ----
    const bool need_mask = (tok0 + kTok - 1 > min_lim) || bad0 || bad1;
    pvec8 pop[NQT];
    pvec8 pop_lo[kSplitP ? NQT : 1];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = sc[qt][e >> 2][e & 3] * c_log2;
      if (need_mask) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = tok0 + 16 * (e >> 2) + 4 * j + (e & 3);
          bool vis;
          if constexpr (TREE)
            vis = t < uEnd && (t < draft0 || (((uint32_t)tree[qt] >> ((t - draft0) & 31)) & 1u));
          else
            vis = t <= lim[qt];
          x[e] = (vis && !((e >> 2) ? bad1 : bad0)) ? x[e] : -INFINITY;
        }
      }
      float mloc = x[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mloc = fmaxf(mloc, x[e]);
      mloc = wave_max_xor16_32(mloc);
      // Lazy rescale: the reference max m_run only moves when some column's
      // block max exceeds it by more than kRescaleLog2 (or it is still -inf).
      // P and l always use the same m_run, so the result is exact up to
      // rounding; p stays below 2^kRescaleLog2 (f16 range).
      if (__any(mloc > m_run[qt] + kRescaleLog2)) {
        const float m_new = fmaxf(m_run[qt], mloc);
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_use);
        l_run[qt] *= alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[qt][t] *= alpha;
        m_run[qt] = m_new;
      }
      const float m_use = (m_run[qt] == -INFINITY) ? 0.0f : m_run[qt];
      float psum = 0.0f;
      i32x4 pw, pw_lo;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(x[e] - m_use);
        const float p1 = __builtin_amdgcn_exp2f(x[e + 1] - m_use);
        psum += p0 + p1;
        pw[e >> 1] = pack2<PT>(p0, p1);
        if constexpr (kSplitP) {
          if constexpr (std::is_same<PT, __bf16>::value) {
            // bf16 -> f32 is exact: the halves are the top 16 bits of an f32
            const uint32_t w = (uint32_t)pw[e >> 1];
            pw_lo[e >> 1] =
                pack2<PT>(p0 - __builtin_bit_cast(float, w << 16), p1 - __builtin_bit_cast(float, w & 0xffff0000u));
          } else {
            // p - hi straight from the packed word's halves: one mix
            // instruction per element instead of a widening and a subtraction.
            const int h = pw[e >> 1];
            pw_lo[e >> 1] = pack2<PT>(sub_half<0>(h, p0), sub_half<1>(h, p1));
          }
        }
      }
      pop[qt] = __builtin_bit_cast(pvec8, pw);
      if constexpr (kSplitP) pop_lo[qt] = __builtin_bit_cast(pvec8, pw_lo);
      l_run[qt] += psum;
    }
    // ---- O^T += V^T . P^T ----
    // d tile t (0 <= t < D/16) holds dims 8*(lane%16) + t (D = 128) or
    // 4*(lane%16) + t (D = 64); k slot i of the V^T and P^T operands is
    // token 16*(i/4) + 4*(lane/16) + i%4 of the block.
#pragma unroll
    for (int tp2 = 0; tp2 < NT; tp2 += 2) {
      i32x4 wa, wb;
      if constexpr (KT != 1) {
        // d tiles tp2, tp2+1 use byte pair (c, c + 1), c = tp2 % 4, of dword tp2 / 4.
        // One byte permute interleaves tokens e and e + 1 (bytes w0.c, w1.c,
        // w0.c+1, w1.c+1), and each half of the result converts straight to an
        // f16 pair (token e, token e + 1) of one dim: 3 VALU instructions per
        // four elements, against 4 through fp32.  v_perm_b32 selectors 0-3 pick
        // bytes of its second operand, 4-7 of its first.
        const uint32_t sel = (tp2 & 3) ? 0x03070206u : 0x01050004u;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          int w0, w1;
          if constexpr (D == 128) {
            w0 = r.v[e][tp2 >> 2];
            w1 = r.v[e + 1][tp2 >> 2];
          } else {
            w0 = r.v[e];
            w1 = r.v[e + 1];
          }
          const int x = (int)__builtin_amdgcn_perm((uint32_t)w0, (uint32_t)w1, sel);
          wa[e >> 1] = cvt_pk_f16<KT == 2>(x, false);
          wb[e >> 1] = cvt_pk_f16<KT == 2>(x, true);
        }
      } else {
        // d tiles tp2, tp2+1 are the low and high halves of dword tp2 / 2:
        // pair the halves of tokens (0, 1) and (2, 3); slots 4-7 are empty
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const uint32_t w0 = (uint32_t)r.v[e][tp2 >> 1];
          const uint32_t w1 = (uint32_t)r.v[e + 1][tp2 >> 1];
          wa[e >> 1] = (int)((w0 & 0xffffu) | (w1 << 16));
          wb[e >> 1] = (int)((w0 >> 16) | (w1 & 0xffff0000u));
        }
        wa[2] = wa[3] = 0;
        wb[2] = wb[3] = 0;
      }
      const pvec8 va = __builtin_bit_cast(pvec8, wa);
      const pvec8 vb = __builtin_bit_cast(pvec8, wb);
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        acc[qt][tp2] = mfma16(va, pop[qt], acc[qt][tp2]);
        acc[qt][tp2 + 1] = mfma16(vb, pop[qt], acc[qt][tp2 + 1]);
        if constexpr (kSplitP) {
          acc[qt][tp2] = mfma16(va, pop_lo[qt], acc[qt][tp2]);
          acc[qt][tp2 + 1] = mfma16(vb, pop_lo[qt], acc[qt][tp2 + 1]);
        }
      }
    }
  }

  // Epilogue: this lane holds column 16*qt + lane%16, dims [DPL*j, DPL*j + DPL).
  // direct: the unit covered the whole sequence; write the output and the
  // LSE (and, with a workspace, mark split slot 0 of the row +inf for the
  // merge).  Otherwise write the fp32 (or fp16) partial (O / l, m, l) of query
  // row i at workspace row slot_row * q_len + i, split slot_split.
  // KERNARG: read the output pointers and strides at the epilogue from the
  // kernel's argument segment (the partial kernel's only argument) instead of
  // keeping them in scalar registers across the block loop.  With one block
  // in flight this halves the scalar spills into VGPR lanes and their reloads
  // in every block (long units: config 4 84.8 -> 83.7 us); with two blocks the
  // epilogue's extra scalar round trip costs more on the short units it
  // serves (config 3 +0.5 us), so those kernels keep the registers.
  template <bool KERNARG>
  __device__ __forceinline__ void finish(const PartialParams &p, int b, int kvh, bool direct, int64_t slot_row,
                                         int64_t slot_split, bool mark_final, float v_scale, int n16, int j,
                                         char *kx) {
    if constexpr (KERNARG) {
      typedef const __attribute__((address_space(4))) PartialParams *KernargParams;
      KernargParams kp = (KernargParams)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(kp));  // no reuse of values loaded before this point
      finish_with(kp, b, kvh, direct, slot_row, slot_split, mark_final, v_scale, n16, j, kx);
    } else {
      finish_with(&p, b, kvh, direct, slot_row, slot_split, mark_final, v_scale, n16, j, kx);
    }
  }
  // Whole-line epilogue for fp32 partial rows (kKLines kernels, D = 128),
  // through the wave's LDS rows kx.  Each lane holds 32 contiguous dims of
  // one column; written straight out, every store instruction would put
  // 16-byte pieces into ~28 different 128-byte lines.  Instead 8 columns at a
  // time go to LDS as the 512-byte rows they form in memory (padded by 16
  // bytes so that the columns written together fall in distinct banks), and
  // are read back 16 bytes per lane in row order: every 8 consecutive lanes
  // store one whole line.  The rows are the wave's own (its K pass of the
  // next block writes them only after these reads, in program order).
  template <typename PP>
  __device__ __forceinline__ void finish_staged(PP pp, int64_t slot_row, int64_t slot_split, int kvh, float v_scale,
                                                int n16, int j, char *kx) {
    constexpr int kRow = 4 * D;       // bytes per fp32 row
    constexpr int kRs = kRow + 16;    // LDS row stride
    constexpr int kCols = 8;          // columns per pass (4608 bytes of rows)
    const int q_len = pp->q_len;
    const int mcols = pp->group * q_len;
    const int lane = n16 + 16 * j;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const float l_tot = wave_sum_xor16_32(l_run[qt]);
      const float inv = (l_tot > 0.0f) ? v_scale / l_tot : 0.0f;
      const int col = 16 * qt + n16;
      if (j == 0 && col < mcols) {
        const int g = col / q_len;
        const int i = col - g * q_len;
        const int64_t h = (int64_t)kvh * pp->group + g;
        const int64_t prow = slot_row * q_len + i;
        pp->pm[prow * pp->pm_srow + h * pp->pm_shead + slot_split * pp->pm_ssplit] = m_run[qt];
        pp->pl[prow * pp->pl_srow + h * pp->pl_shead + slot_split * pp->pl_ssplit] = l_tot;
      }
      const int ncols = min(16, mcols - 16 * qt);
      for (int c0 = 0; c0 < ncols; c0 += kCols) {
        if (n16 >= c0 && n16 < c0 + kCols && n16 < ncols) {
          char *rowp = kx + (n16 - c0) * kRs;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
#pragma unroll
            for (int t = 0; t < NT; t += 4)
              *reinterpret_cast<f32x4 *>(rowp + 4 * (DPL * j + rr * NT + t)) =
                  f32x4{acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv, acc[qt][t + 2][rr] * inv,
                        acc[qt][t + 3][rr] * inv};
          }
        }
        const int nbytes = min(kCols, ncols - c0) * kRow;
        for (int o0 = 0; o0 < nbytes; o0 += 1024) {
          const int o = o0 + 16 * lane;
          if (o < nbytes) {
            const int c = o / kRow;
            const int w = o - c * kRow;
            const i32x4 v = *reinterpret_cast<const i32x4 *>(kx + c * kRs + w);
            const int gc = 16 * qt + c0 + c;
            const int g = gc / q_len;
            const int i = gc - g * q_len;
            const int64_t h = (int64_t)kvh * pp->group + g;
            char *dst = reinterpret_cast<char *>(pp->po) +
                        ((slot_row * q_len + i) * pp->po_srow + h * pp->po_shead + slot_split * pp->po_ssplit) * 4;
            *reinterpret_cast<i32x4 *>(dst + w) = v;
          }
        }
      }
    }
  }
  template <typename PP>
  __device__ __forceinline__ void finish_with(PP pp, int b, int kvh, bool direct, int64_t slot_row,
                                              int64_t slot_split, bool mark_final, float v_scale, int n16, int j,
                                              char *kx) {
    // Whole-line stores through LDS rows pay for fp32 partials of two query
    // tiles (config 5 partial kernel 99.8 -> 97.7 us); with one tile, or 16-bit
    // rows, the direct column stores are as fast or faster (config 3: 46.7 vs
    // 47.6 us with fp16 partials).
    if constexpr (kKLines && D == 128 && NQT > 1) {
      if (!direct && pp->po_kind == 0) {
        finish_staged(pp, slot_row, slot_split, kvh, v_scale, n16, j, kx);
        return;
      }
    }
    const int q_len = pp->q_len;
    const int mcols = pp->group * q_len;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const float l_tot = wave_sum_xor16_32(l_run[qt]);
      const int col = 16 * qt + n16;
      if (col >= mcols) continue;
      const float inv = (l_tot > 0.0f) ? v_scale / l_tot : 0.0f;
      const int g = col / q_len;
      const int i = col - g * q_len;
      const int64_t h = (int64_t)kvh * pp->group + g;
      if (direct) {
        const int64_t row = (int64_t)b * q_len + i;
        QT *dst = reinterpret_cast<QT *>(pp->out) + row * pp->o_srow + h * pp->o_shead + DPL * j;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          if constexpr (D == 128) {
            i32x4 w;
#pragma unroll
            for (int t = 0; t < NT; t += 2) w[t >> 1] = pack2<QT>(acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv);
            *reinterpret_cast<i32x4 *>(dst + rr * NT) = w;
          } else {
            i32x2 w;
#pragma unroll
            for (int t = 0; t < NT; t += 2) w[t >> 1] = pack2<QT>(acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv);
            *reinterpret_cast<i32x2 *>(dst + rr * NT) = w;
          }
        }
        if (j == 0 && pp->lse) {
          const float m = (m_run[qt] == -INFINITY) ? 0.0f : m_run[qt];
          // v_log_f32 is log2
          pp->lse[row * pp->lse_srow + h * pp->lse_shead] = (l_tot > 0.0f) ? kLn2 * (m + __builtin_amdgcn_logf(l_tot)) : -INFINITY;
        }
        if (j == 0 && mark_final) pp->pm[row * pp->pm_srow + h * pp->pm_shead] = INFINITY;  // merge: already final
      } else {
        const int64_t prow = slot_row * q_len + i;
        const int64_t po_idx = prow * pp->po_srow + h * pp->po_shead + slot_split * pp->po_ssplit + DPL * j;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          if (pp->po_kind == 0) {
            float *dst = reinterpret_cast<float *>(pp->po) + po_idx + rr * NT;
#pragma unroll
            for (int t = 0; t < NT; t += 4)
              *reinterpret_cast<f32x4 *>(dst + t) = f32x4{acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv,
                                                          acc[qt][t + 2][rr] * inv, acc[qt][t + 3][rr] * inv};
          } else {
            // 16-bit partials: 2 bytes per element at the same element offsets
            _Float16 *dst = reinterpret_cast<_Float16 *>(pp->po) + po_idx + rr * NT;
            const bool bf = pp->po_kind == 2;
            if constexpr (D == 128) {
              i32x4 w;
#pragma unroll
              for (int t = 0; t < NT; t += 2)
                w[t >> 1] = bf ? pack2<__bf16>(acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv)
                               : pack2<_Float16>(acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv);
              *reinterpret_cast<i32x4 *>(dst) = w;
            } else {
              i32x2 w;
#pragma unroll
              for (int t = 0; t < NT; t += 2)
                w[t >> 1] = bf ? pack2<__bf16>(acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv)
                               : pack2<_Float16>(acc[qt][t][rr] * inv, acc[qt][t + 1][rr] * inv);
              *reinterpret_cast<i32x2 *>(dst) = w;
            }
          }
        }
        if (j == 0) {
          pp->pm[prow * pp->pm_srow + h * pp->pm_shead + slot_split * pp->pm_ssplit] = m_run[qt];
          pp->pl[prow * pp->pl_srow + h * pp->pl_shead + slot_split * pp->pl_ssplit] = l_tot;
        }
      }
    }
  }
};

// Splits of sequence b taken by the static first round: workgroup w starts
// on slot w of the split-major numbering (sequence w % B, split w / B).
__device__ __forceinline__ int static_splits(int b, int G, int B) { return b < G ? (G - 1 - b) / B + 1 : 0; }

// Persistent, page-major partial kernel: a continuous K/V block stream per wave.
//
// Work items are (sequence, split) pairs; a unit is one KV head of an item.
// Wave w of a workgroup owns KV heads w, w + W, ... of every item the
// workgroup takes, so the waves of an item read the interleaved per-head
// pieces of the same 16-token pages together and the NHD page is fetched as
// a whole.
//
// Item order.  Workgroup w first takes slot w of the split-major numbering
// (sequence w % B, split w / B), which needs no prefix: its page ids and the
// sequence length are fetched together, so the first K/V loads leave after
// one round trip.  The remaining items form the queue: with at most
// kMaxCompactBatch sequences (compact mode) queue index c is decoded through
// an LDS prefix of the per-sequence counts of items left after the static
// round (no empty items); otherwise c continues the split-major numbering and
// the claiming wave skips its holes.  Workgroups claim queue items one at a
// time from one counter, in order.  An item's successor is
// claimed only a few blocks before the item ends (a workgroup never holds an
// unstarted item for long, so the queue stays balanced to the end) and is
// published to all waves early enough for the tail of the item to stream its
// first blocks.
//
// Block stream.  A wave keeps NB 32-token blocks of raw fp8 K/V in registers
// (two; one for long units, where half the bytes in flight still fill the
// memory system and queue half as long).  After computing block k of unit U
// it refills that buffer with stream position k + NB: U's own block, or one
// of the first NB blocks of the next unit N, whose page ids (and, for one
// query tile, query operand) are loaded a few blocks before U ends.  The
// stream never drains between units; block k of a unit sits in buffer
// (k + par) % NB, par carried over from unit to unit.
//
// An item of a single-split sequence writes the final output and LSE (and
// marks split slot 0 with +inf for the merge); any other item writes its
// fp32 partial (o / l, m, l) at its split slot.
template <typename QT, int KT, int D, int NQT, bool TREE, int NB>
__global__ __launch_bounds__(512) void pd_fp8_partial(PartialParams p) {
  typedef KvUnit<QT, KT, D, NQT, TREE, KT != 1 && D == 128 && (NB == 1 || NQT == 1)> U;
  typedef typename U::qvec8 qvec8;
  typedef typename U::Block Block;
  constexpr int kTok = U::kTok;            // tokens per block
  constexpr int kLeadMul = 32 / kTok;      // hand-off leads in 32-token units
  constexpr int NS = U::NS;
  // One query tile: the next unit's query operand is prefetched into a second
  // register set.  Two tiles: it is loaded once the current unit's last block
  // has been computed.
  constexpr bool kQPrefetch = NQT == 1;
  static_assert(NB == 1 || NB == 2, "one or two blocks in flight per wave");
  constexpr int kNeedLead = need_lead(NB);
  constexpr int kPublishLead = publish_lead(NB);
  constexpr int kClaimLead = claim_lead(NB);

  extern __shared__ int s_dyn[];  // compact mode: s_prefix[B + 1], s_len[B]
  __shared__ int s_pub[2][2][3];  // per wave group: published item (b, s, L); b = -1: none
  __shared__ int s_cap;  // poll limit of the hand-off waits (p.spin_cap)
  __shared__ int s_tag;  // the launch's work-queue tag
  __shared__ int s_seq[2][2];     // per wave group: item number of the slot's contents
  __shared__ int s_ack[2][2];     // per wave group: waves other than 0 that have read the slot
  __shared__ int s_prefix_ready;
  // per-wave LDS rows of the whole-line K pass (kKLines)
  __shared__ __attribute__((aligned(16))) char s_kx[U::kKLines ? kMaxWaves * U::kKxBytes : 16];

  // Two items per workgroup (p.paired, instances with one query tile, two
  // blocks in flight and the whole-line K pass): wave group grp (waves
  // [grp W, grp W + W)) runs virtual workgroup grp * gridDim.x + blockIdx.x
  // of the schedule below, with its own hand-off words; the LDS prefix is
  // shared.  Both items of a CU then share one dispatch and one LDS.
  constexpr bool kPairable = U::kKLines && NQT == 1 && NB == 2 && !TREE;
  const bool paired = kPairable && p.paired != 0;
  const int nw_all = blockDim.x >> 6;
  const int nwaves = paired ? nw_all >> 1 : nw_all;  // waves per item
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int grp = paired && wave >= nwaves ? 1 : 0;
  const int gwave = wave - grp * nwaves;  // the wave's index in its group: its first KV head
  const int vblk = grp * (int)gridDim.x + (int)blockIdx.x;
  const int n16 = lane & 15;
  const int j = lane >> 4;
  char *const kx = s_kx + (U::kKLines ? wave * U::kKxBytes : 0);
  const int q_len = p.q_len;
  const int B = p.batch;
  const int S = p.split_size;
  const int G = (paired ? 2 : 1) * (int)gridDim.x;  // virtual workgroups
  const int hpw = p.num_kv_heads / nwaves;  // units per item and wave
  const bool compact = p.compact != 0;
  // Items beyond the split-major slots of the grid go through the queue.
  // Then, in compact mode, only workgroups [0, G1), G1 = min(2B, G/2), start
  // on a split-major slot -- one per CU, the first workgroup dispatched to
  // each: split 0 of every sequence, then split 1 of sequences [0, G1 - B).
  // Its page ids and length load together, so it needs no prefix.
  // Workgroup w >= G1 starts on queue item w - G1 of the compact numbering
  // without a claim.  Its page ids need the LDS prefix first, but as the
  // second workgroup on its CU its first loads would queue behind the first
  // one's K/V burst anyway.  A static slot that is a hole (split 1 of a
  // one-split sequence) takes queue item G - G1 + its rank among the holes,
  // again without a claim, so atomic claims number the items after those
  // G - G1 + H (H holes) and are made only when the queue holds more.
  // (Config 3, B = 128 on a 512-workgroup grid: every CU starts a static
  // item at once, and most input sets need no claim: partial kernel 45.2 ->
  // 44.3 us against split 0 alone as the static round, 45.7 with claims.)
  const bool queued = (int64_t)G < (int64_t)B * p.num_splits;
  const int G1 = (compact && queued) ? min(2 * B, (G + 1) / 2) : G;
  int *s_prefix = s_dyn;      // s_prefix[b]: queue items of sequences < b
  int *s_len = s_dyn + B + 1;  // clamped length of sequence b
  int *s_holes = s_dyn + 2 * B + 1;  // static slots that are holes (split 1 of a one-split sequence)

  // ---- per-wave helpers ----
  auto n_blocks = [&](int s, int L) {
    const int start = s * S;
    const int tiles = max(0, (min(start + S, L) - start + kPage - 1) / kPage);
    return KT != 1 ? (tiles + 1) >> 1 : tiles;
  };
  // Sequence b's page list and its length (a block-table row, or the CSR
  // slice; l20_paged_decode.cu:205-208).
  auto row_of = [&](int b) -> const int32_t * {
    return p.indptr ? p.bt + uniform_ld(p.indptr, b) : p.bt + (int64_t)b * p.bt_srow;
  };
  auto pages_of = [&](int b) {
    return p.indptr ? uniform_ld(p.indptr, b + 1) - uniform_ld(p.indptr, b) : p.bt_pages;
  };
  // Virtual 16-token page of tile T of a page list; -1 for an entry outside
  // the cache (checked in 64 bits, before any product can wrap).
  auto tile_page = [&](const int32_t *row, int T) -> int {
    const int m = p.page_mult;
    if (__builtin_expect(m == 1, 1)) {
      const int e = row[T];
      return (e >= 0 && (int64_t)e < p.num_pages) ? e : -1;
    }
    const int q = (int)__umulhi((unsigned int)T, p.page_magic);  // T / m
    const int e = row[q];
    const int64_t v = (int64_t)e * m + (T - q * m);
    return (e >= 0 && v < p.num_pages) ? (int)v : -1;
  };
  // Page ids of split s of sequence b: lane t -> tile t (a split has <= 64
  // tiles); -1 for tiles past the split, past the page list, and for
  // out-of-range ids.
  auto load_pid = [&](int b, int s, int L) {
    const int start = s * S;
    const int tiles = max(0, (min(start + S, L) - start + kPage - 1) / kPage);
    const int avail = pages_of(b) * p.page_mult - start / kPage;
    int v = -1;
    if (lane < tiles && lane < avail) {
      v = tile_page(row_of(b), start / kPage + lane);
    }
    return v;
  };
  auto load_tree = [&](int b, int (&dst)[TREE ? NQT : 1]) { U::load_tree(p, b, dst, n16); };
  auto load_q = [&](int b, int kvh, qvec8 (&dst)[NQT][NS]) { U::load_q(p, b, kvh, dst, n16, j); };
  // parts: 1 = the K loads, 2 = the V loads, 3 = both (a constant at every call)
  auto load_block = [&](Block &r, int pid, int kvh, int blk, int parts = 3) {
    U::load_block(p, r, pid, kvh, blk, parts, n16, j);
  };
  auto load_pages = [&](Block &r, const int (&pg)[2], int kvh, int parts = 3) {
    U::load_pages(p, r, pg, kvh, parts, n16, j);
  };

  // ---- stream state (wave-uniform except the VGPR operands) ----
  Block buf[NB];
  qvec8 qop[NQT][NS];
  qvec8 qopN[kQPrefetch ? NQT : 1][NS];
  int pidU = -1;
  int treeU[TREE ? NQT : 1];                    // ancestor words of the current unit
  int treeN[TREE && kQPrefetch ? NQT : 1];      // ... and of the next (prefetched with its query)
  int par = 0;         // block k of the current unit is in buf[(k + par) & 1]
  int issuedU = 0;     // blocks of the current unit already loading
  bool u_loaded = false;  // page ids and query of the current unit are loading

  // ---- static first item: slot vblk of the split-major numbering ----
  int cb = (int)((unsigned)vblk % (unsigned)B);
  int cs = (int)((unsigned)vblk / (unsigned)B);
  int cL = 0;
  if (vblk >= G1) {
    cb = -2;  // starts on queue item vblk - G1
  } else {
    // The query and tree words leave with the page ids and the length, before
    // any K/V load: the wait for the ids covers them, so no step waits on a
    // query load issued behind the stream.  (Issued after the first blocks'
    // K/V, they were the most recent loads when the block loop began, and the
    // loop's static wait before the score product drained every load in flight
    // on each of its iterations.)  The ids are masked to the split once the
    // length is known.
    load_q(cb, gwave, qop);
    load_tree(cb, treeU);
    const int start = cs * S;
    const int spec = min(S / kPage, pages_of(cb) * p.page_mult - start / kPage);
    int v = -1;
    if (lane < spec) v = tile_page(row_of(cb), start / kPage + lane);
    cL = clamped_len(p, cb);
    if (cs < splits_of_len(cL, S)) {
      const int tiles = max(0, (min(start + S, cL) - start + kPage - 1) / kPage);
      pidU = (lane < tiles && lane < spec && v >= 0 && (int64_t)v < p.num_pages) ? v : -1;
      const int nU = KT != 1 ? (tiles + 1) >> 1 : tiles;
      // Both buffers load, a block past the unit's end reading page 0 (its
      // tiles hold page id -1), so the stream enters its loop with the loads
      // in flight of any later step.
      load_block(buf[0], pidU, gwave, 0);
      if constexpr (NB > 1) load_block(buf[NB - 1], pidU, gwave, 1);
      issuedU = min(nU, NB);
      u_loaded = true;
    } else {
      cb = -2;  // hole: the workgroup starts on the queue
    }
  }

  if (threadIdx.x == 0) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      lds_put(&s_seq[g][0], -1);
      lds_put(&s_seq[g][1], -1);
      lds_put(&s_ack[g][0], nwaves - 1);  // both slots start out consumed
      lds_put(&s_ack[g][1], nwaves - 1);
    }
    lds_put(&s_prefix_ready, 0);
    lds_put(&s_cap, (int)p.spin_cap);
    const uint64_t dp = (uint64_t)__builtin_amdgcn_dispatch_ptr();
    lds_put(&s_tag, (int)(p.launch_tag * 0x9E3779B1u + (unsigned int)(dp >> 6) * 0x85EBCA77u +
                          (unsigned int)(dp >> 38)));
  }
  __syncthreads();

  // ---- the queue (wave 0 only) ----
  // Compact mode: s_prefix / s_len, built by the last wave while its first
  // blocks load and read only by wave 0, which waits for s_prefix_ready
  // before its first decode.
  auto build_prefix = [&]() {
    const int per = (B + 63) >> 6;  // sequences per lane, <= 64
    int sum = 0, holes = 0;
    for (int e0 = 0; e0 < per; e0 += 8) {
      int lv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = lane * per + e0 + e;
        lv[e] = (e0 + e < per && idx < B) ? p.seq_lens[idx] : 0;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = lane * per + e0 + e;
        if (e0 + e < per && idx < B) {
          const int L = max(0, min(lv[e], p.l_cap));
          s_len[idx] = L;
          sum += max(0, splits_of_len(L, S) - static_splits(idx, G1, B));
          holes += (idx < G1 - B && splits_of_len(L, S) <= 1) ? 1 : 0;
        }
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) holes += __shfl_xor(holes, off);
    if (lane == 0) s_holes[0] = holes;
    int incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    int run = incl - sum;
    for (int e = 0; e < per; ++e) {
      const int idx = lane * per + e;
      if (idx < B) {
        run += max(0, splits_of_len(s_len[idx], S) - static_splits(idx, G1, B));
        s_prefix[idx + 1] = run;
      }
    }
    if (lane == 0) s_prefix[0] = 0;
  };
  auto queue_total = [&]() -> int64_t {
    if (compact) return lds_uniform(s_prefix, B);
    return max((int64_t)0, (int64_t)B * p.num_splits - G);
  };
  // Queue index -> item (b, s, L); false for a hole of the split-major numbering.
  int db = -1, ds = 0, dL = 0;
  auto decode = [&](int64_t c) {
    if (compact) {
      // Last b with s_prefix[b] <= c (the prefix is non-decreasing and
      // s_prefix[0] = 0): two ballot rounds, chunks of ceil(B / 64).
      const int ci = (int)c;
      const int chunk = (B + 63) >> 6;
      int idx = lane * chunk;
      const uint64_t m1 = __ballot(idx < B && s_prefix[idx] <= ci);
      const int base = (__popcll(m1) - 1) * chunk;
      idx = base + lane;
      const uint64_t m2 = __ballot(lane < chunk && idx < B && s_prefix[idx] <= ci);
      const int b = base + __popcll(m2) - 1;
      db = b;
      ds = static_splits(b, G1, B) + (ci - lds_uniform(s_prefix, b));
      dL = lds_uniform(s_len, b);
      return true;
    }
    const int64_t slot = (int64_t)G + c;
    const int b = (int)(slot % B);
    const int s = (int)(slot / B);
    const int L = clamped_len(p, b);
    if (s >= splits_of_len(L, S)) return false;
    db = b;
    ds = s;
    dL = L;
    return true;
  };

  // ---- next-item hand-off ----
  // Item t's successor is claimed by wave 0 late in its last unit (claim
  // point) and resolved and published in LDS slot t & 1 a few blocks later
  // (checkpoint).  The other waves poll the slot from their own checkpoint
  // on and wait for it only when they need the successor's page ids (two
  // blocks before their unit ends); they then start prefetching it.  No
  // barrier separates items: each reader acknowledges the slot, and wave 0
  // rewrites a slot only after every other wave has acknowledged it.
  // wave 0: a claim is in flight (a workgroup past the split-major round
  // holds queue item blockIdx.x - G1 as if claimed; atomic claims number
  // the items after those)
  // claim: the counter's value before the atomic claim (item = its low half
  // + G - G1 + H), or for a pre-assigned item its number less 2^30, a
  // negative low half (no flag: a boolean carried through the item loop
  // cost the kernel ~60 SGPRs of spills).
  uint64_t claim = vblk >= G1 ? (uint64_t)(uint32_t)(vblk - G1 - (1 << 30)) : 0u;
  bool claimed = vblk >= G1;
  // wave 0: the queue may still hold items (never, when the static round
  // covers every slot: then no workgroup claims)
  bool more = queued;
  int t_item = 0;
  int nb = -1, ns = 0, nL = 0;
  auto issue_claim = [&]() {
    const unsigned int tag = (unsigned int)__builtin_amdgcn_readfirstlane(lds_poll(&s_tag));
    if (lane == 0)
      claim = __hip_atomic_fetch_add(&g_pd_queue[p.queue_slot][0], 1ull | ((uint64_t)tag << 32), __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    claimed = true;
  };
  // Compact mode: atomic claims only when the queue holds items beyond the
  // pre-assigned ones (a launch constant, so every workgroup decides alike:
  // either all claim until a claim fails, or none touches the counter).  At
  // config 3 the claims' latency depends on where the counter line sits in
  // HBM (partial kernel 45.4-48.0 us over 64 positions), and most of its
  // input sets need no claim at all.
  auto hole_count = [&]() { return compact ? lds_uniform(s_holes, 0) : 0; };
  auto claims_needed = [&]() { return !compact || queue_total() > (int64_t)(G - G1) + hole_count(); };
  auto claim_point = [&]() {
    if (gwave == 0 && more && !claimed) {
      // without the prefix yet, resolve decides after its prefix wait
      if (compact && !__builtin_amdgcn_readfirstlane(lds_acquire(&s_prefix_ready))) return;
      if (claims_needed()) issue_claim();
    }
  };
  // Bounded polling: a wait loop counts its polls and stops at the limit;
  // past the loop, a wait that gave up records its error code.
  // The poll limit is copied into LDS at the workgroup's start and read from
  // there when a wait starts: no register holds it across the block stream,
  // and no wait path touches memory.  (Read from device memory, or again from
  // the argument segment, the limit arrived only after the workgroup's K/V
  // burst: at config 3 the waves that waited for their first item saw it ~3
  // us late.)
  auto spin_cap = [&]() { return (unsigned int)__builtin_amdgcn_readfirstlane(lds_poll(&s_cap)); };
  auto record_give_up = [&](unsigned int code) {
    if (lane == 0) __hip_atomic_fetch_or(&g_pd_error[p.queue_slot], code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  // Wave 0: the next item into (db, ds, dL); db = -1 when none is left.
  auto resolve_claim = [&]() {
    db = -1;
    if (!more) return;
    if (compact) {
      unsigned int polls = 0;
      if (!__builtin_amdgcn_readfirstlane(lds_acquire(&s_prefix_ready))) {
        const unsigned int cap = spin_cap();
        while (!__builtin_amdgcn_readfirstlane(lds_acquire(&s_prefix_ready)) && ++polls < cap)
          __builtin_amdgcn_s_sleep(1);
        if (polls < cap) polls = 0;
      }
      if (__builtin_expect(polls != 0, 0)) {
        record_give_up(L20_PD_DEVERR_PREFIX_WAIT);
        more = false;
        return;
      }
    }
    if (!claimed && compact && t_item == 0 && cb == -2 && vblk < G1) {
      // The static slot was a hole (split 1 of a one-split sequence): the
      // hole takes pre-assigned queue item G - G1 + its rank among holes.
      const int bh = vblk - B;
      int h = 0;
      for (int base = 0; base < bh; base += 64) {
        const int idx = base + lane;
        h += __popcll(__ballot(idx < bh && splits_of_len(s_len[idx], S) <= 1));
      }
      claim = (uint64_t)(uint32_t)((G - G1) + h - (1 << 30));
      claimed = true;
    }
    if (!claimed) {
      if (!claims_needed()) {
        more = false;
        return;
      }
      issue_claim();
    }
    const int64_t Q = queue_total();
    for (;;) {
      const unsigned int lo = __builtin_amdgcn_readfirstlane((unsigned int)claim);
      const unsigned int hi = __builtin_amdgcn_readfirstlane((unsigned int)(claim >> 32));
      const bool atomic = (int)lo >= 0;
      const int64_t c = atomic ? (int64_t)lo + (G - G1) + hole_count() : (int64_t)(int)lo + (1 << 30);
      claimed = false;
      // (c < 0: a counter left flagged for ~2^31 claims without a clear; its
      // low half now reads as a pre-assigned item)
      if (c < 0 || (atomic && hi != lo * (unsigned int)__builtin_amdgcn_readfirstlane(lds_poll(&s_tag)))) {
        record_give_up(L20_PD_DEVERR_QUEUE_SHARED);
        more = false;
        return;
      }
      if (c >= Q) {
        more = false;
        // The launch's last atomic claim: no other atomic on the counter
        // follows.  When claims are made at all, every workgroup makes
        // exactly one failing atomic claim (no pre-assigned item fails then),
        // so the last atomic returns Q + G - 1 (after the G - G1 + H offset).
        if (atomic && lane == 0 && c == Q + G - 1) g_pd_queue[p.queue_slot][0] = 0ull;
        // A clean launch never claims past Q + G - 1 (a second check, for a
        // tag that happens to match).
        if (c > Q + G - 1) record_give_up(L20_PD_DEVERR_QUEUE_SHARED);
        return;
      }
      if (decode(c)) return;
      issue_claim();  // a hole of the split-major numbering
    }
  };
  auto resolve = [&]() { resolve_claim(); };
  // Returns true once (nb, ns, nL) holds item t_item's successor.  Wave 0
  // always completes; another wave returns false when `wait` is unset and
  // the slot is not published yet.
  auto checkpoint = [&](bool wait) {
    const int slot = t_item & 1;
    if (gwave == 0) {
      resolve();
      unsigned int polls = 0;
      if (__builtin_amdgcn_readfirstlane(lds_acquire(&s_ack[grp][slot])) < nwaves - 1) {
        const unsigned int cap = spin_cap();
        while (__builtin_amdgcn_readfirstlane(lds_acquire(&s_ack[grp][slot])) < nwaves - 1 && ++polls < cap)
          __builtin_amdgcn_s_sleep(1);
        if (polls < cap) polls = 0;
      }
      // A wave that never acknowledged the slot's previous item may read the
      // new one instead (valid indices, wrong results, the error recorded).
      if (__builtin_expect(polls != 0, 0)) record_give_up(L20_PD_DEVERR_ACK_WAIT);
      if (lane == 0) {
        lds_put(&s_ack[grp][slot], 0);
        lds_put(&s_pub[grp][slot][0], db);
        lds_put(&s_pub[grp][slot][1], ds);
        lds_put(&s_pub[grp][slot][2], dL);
        // Release: the reset and the item fields are visible to a wave that
        // reads this item number with acquire.
        lds_publish(&s_seq[grp][slot], t_item);
      }
      nb = db;
      ns = ds;
      nL = dL;
      return true;
    }
    if (__builtin_amdgcn_readfirstlane(lds_acquire(&s_seq[grp][slot])) != t_item) {
      if (!wait) return false;
      const unsigned int cap = spin_cap();
      unsigned int polls = 0;
      while (__builtin_amdgcn_readfirstlane(lds_acquire(&s_seq[grp][slot])) != t_item && ++polls < cap)
        __builtin_amdgcn_s_sleep(1);
      if (__builtin_expect(polls >= cap, 0)) {
        record_give_up(L20_PD_DEVERR_PUBLISH_WAIT);
        nb = -1;  // this wave stops after its current unit
        return true;
      }
    }
    nb = __builtin_amdgcn_readfirstlane(lds_poll(&s_pub[grp][slot][0]));
    ns = __builtin_amdgcn_readfirstlane(lds_poll(&s_pub[grp][slot][1]));
    nL = __builtin_amdgcn_readfirstlane(lds_poll(&s_pub[grp][slot][2]));
    // Release: the reads above complete before wave 0 can see the acknowledgement.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) __hip_atomic_fetch_add(&s_ack[grp][slot], 1, L20_PD_LDS_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    return true;
  };

  if (compact && more && wave == nw_all - 1) {
    build_prefix();
    // Every lane stores the flag with release: each lane's own table entries
    // are then visible to a wave whose acquire load sees the flag.
    lds_publish(&s_prefix_ready, 1);
  }

  int hh = 0;
  while (cb != -1) {
    if (cb < 0) checkpoint(true);  // the static item was a hole
    if (cb >= 0) {
      const int kvh = gwave + nwaves * hh;
      const int b = cb;
      const int L = cL;
      const int split = cs;
      const int uStart = split * S;
      const int uEnd = min(uStart + S, L);
      const int nU = n_blocks(split, L);
      const int n_b = splits_of_len(L, S);
      const bool direct = n_b == 1;
      const bool has_ws = p.num_splits > 1;
      const bool last = hh + 1 == hpw;  // the item's successor follows this unit
      if (!u_loaded) {
        pidU = load_pid(b, split, L);
        load_q(b, kvh, qop);
        load_tree(b, treeU);
        issuedU = 0;
      }
      // Top up the unit's first NB blocks (a block past the unit's end reads
      // page 0: its tiles hold page id -1), so every path issues the same loads.
      auto top_up = [&](Block &r, int blk) { load_block(r, pidU, kvh, blk); };
      if constexpr (NB == 1) {
        if (issuedU < 1) top_up(buf[0], 0);
      } else {
        if (issuedU < 1) {
          if (par) top_up(buf[NB - 1], 0);
          else top_up(buf[0], 0);
        }
        if (issuedU < 2) {
          if (par) top_up(buf[0], 1);
          else top_up(buf[NB - 1], 1);
        }
      }
      // The query (and tree words) must have arrived before the block loop:
      // left pending, their loads sit behind the stream's on some path into
      // the loop, and its static waits before the score product then drain
      // every load in flight on each iteration.  The pin waits for them here,
      // with the first blocks' K/V still in flight.
      pin_operands(qop);
      if constexpr (TREE) pin_words(treeU);

      // ---- the next unit of this wave ----
      bool hasN = false;
      int nKvh = 0, nB = 0, nN = 0, pidN = -1;
      int issuedN = 0;
      auto set_next = [&]() {
        if (!last) {
          hasN = true;
          nB = b;
          nKvh = kvh + nwaves;
          nN = nU;
          pidN = pidU;
        } else if (nb >= 0) {
          hasN = true;
          nB = nb;
          nKvh = gwave;
          nN = n_blocks(ns, nL);
          pidN = load_pid(nb, ns, nL);
        }
        if constexpr (kQPrefetch) {
          if (hasN) {
            load_q(nB, nKvh, qopN);
            load_tree(nB, treeN);
          }
        }
      };
      // In the last unit the successor is claimed kClaimLead blocks and
      // published kPublishLead blocks before the end (at the start of a
      // shorter unit); the first blocks of N leave two blocks before the end.
      const int k_claim = last ? nU - kClaimLead * kLeadMul : -1;
      const int k_pub = last ? nU - kPublishLead * kLeadMul : -1;
      bool n_ready = !last;
      if (last) {
        if (k_claim < 0) claim_point();
        if (k_pub < 0) n_ready = checkpoint(true);
      }
      if (n_ready) set_next();

      const float k_scale = p.k_scale_ph ? uniform_ld(p.k_scale_ph, kvh) : p.k_scale;
      const float v_scale = p.v_scale_ph ? uniform_ld(p.v_scale_ph, kvh) : p.v_scale;
      const float c_log2 = k_scale * p.qk_scale_log2;
      // ---- masking: keys before draft0 are visible to every column; key
      // draft0 + j to draft row i when j <= i (causal) or when bit j of the
      // row's ancestor word is set (TREE) ----
      const int draft0 = L - q_len;  // first key of the newest q_len
      int lim[TREE ? 1 : NQT];       // causal: last visible key of the lane's column
      if constexpr (!TREE) {
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) lim[qt] = min(uEnd - 1, draft0 + (16 * qt + n16) % q_len);
      }
      // the last key that every column sees
      const int min_lim = min(uEnd - 1, TREE ? draft0 - 1 : draft0);

      U st;
      st.reset();
      auto compute_block = [&](Block &r, int blk, auto &&after_scores) {
        st.compute_block(r, pidU, blk, uStart + kTok * blk, uEnd, draft0, lim, min_lim, treeU, qop, c_log2, j, kx,
                         after_scores);
      };

      // Compute block k, then refill its buffer with stream position k + 2:
      // the unit's own block or, in order, the next unit's first two blocks.
      auto step = [&](Block &r, int k) {
        // The refill of r: block k + NB of this unit, or of the next.  With
        // two blocks in flight it is issued in two parts, its K loads as soon
        // as the scores of block k have consumed r.k and its V loads after
        // the V^T.P^T product, so the softmax and PV of block k overlap the
        // refill's K latency (config 3 49.6 -> 49.2 us, bf16 caches 89.1 ->
        // 88.3).  With one block in flight the split cost 0.5-3.9 us (long
        // context, verify, tree), so K and V leave together after the block.
        const int pos = k + NB;
        const bool own = pos < nU;
        const bool nxt = !own && pos - nU == issuedN && issuedN < nN;
        // Every step issues its refill's loads -- a dummy block reading page 0
        // when the stream has nothing left -- from one straight-line sequence:
        // only the page ids are chosen per case.  With the same loads, in the
        // same order, on every path the compiler's load counters wait for r's
        // block alone; refills issued on some paths and not others (or
        // partly merged across the cases) made it wait for every load in
        // flight, the other buffer's refill included, before the next block.
        int pg[2] = {-1, -1};
        int rkvh = kvh;
        if (own) {
          U::block_pages(pidU, pos, pg);
        } else if (nxt) {
          U::block_pages(pidN, issuedN, pg);
          rkvh = nKvh;
        }
        compute_block(r, k, [&]() {
          if constexpr (NB > 1) load_pages(r, pg, rkvh, 1);
        });
        constexpr int kLate = NB > 1 ? 2 : 3;  // the parts left for after the block
        load_pages(r, pg, rkvh, kLate);
        if (nxt) ++issuedN;
        if (k == k_claim) claim_point();
        // From the checkpoint on, poll for the successor; wait for it
        // kNeedLead blocks before the end (its first block is the refill
        // after the next).
        if (!n_ready && k >= k_pub) {
          n_ready = checkpoint(k + kNeedLead >= nU);
          if (n_ready) set_next();
        }
      };
      if constexpr (NB == 1) {
        for (int k = 0; k < nU; ++k) step(buf[0], k);
      } else {
        int k = 0;
        if (par && nU > 0) {
          step(buf[NB - 1], 0);
          k = 1;
        }
        for (; k + 1 < nU; k += 2) {
          step(buf[0], k);
          step(buf[NB - 1], k + 1);
        }
        if (k < nU) step(buf[0], k);
      }
      if constexpr (!kQPrefetch)
        if (hasN) {
          load_q(nB, nKvh, qop);  // qop and treeU are dead once the last block is computed
          load_tree(nB, treeU);
        }

      // ---- epilogue ----
      st.template finish<true>(p, b, kvh, direct, b, split, direct && has_ws, v_scale, n16, j, kx);

      // ---- the next unit inherits the stream ----
      par = (par + nU) % NB;
      pidU = pidN;
      if constexpr (TREE && kQPrefetch) treeU[0] = treeN[0];
      issuedU = issuedN;
      u_loaded = hasN;
      if constexpr (kQPrefetch) {
        if (hasN) {
#pragma unroll
          for (int s = 0; s < NS; ++s) qop[0][s] = qopN[0][s];
        }
      }
      if (hh + 1 < hpw) {
        ++hh;
        continue;
      }
    }
    // ---- item transition (no barrier: see the hand-off above) ----
    hh = 0;
    cb = nb;
    cs = ns;
    cL = nL;
    ++t_item;
  }
  // Every claim of this workgroup has been resolved by now; the counter was
  // reset by the launch's last claim.  No fence: the counter orders nothing
  // else, and the kernel boundary publishes the reset (a fence would write
  // back the XCD's L2).
}

// ---------------------------------------------------------------------------
// LSE merge kernel
// ---------------------------------------------------------------------------
// Eight consecutive partial o/l elements at element offset off, as fp32.  PK
// is a template argument: a run-time choice between the three loads puts a
// branch around each one, and the compiler then waits for every load before
// issuing the next (eight dependent round trips in the narrow merge).
template <int PK>
__device__ __forceinline__ void load_partial8(const void *po, int64_t off, f32x4 &a, f32x4 &b) {
  if constexpr (PK == 0) {
    const float *src = reinterpret_cast<const float *>(po) + off;
    a = *reinterpret_cast<const f32x4 *>(src);
    b = *reinterpret_cast<const f32x4 *>(src + 4);
  } else if constexpr (PK == 1) {
    const f16x8 v = *reinterpret_cast<const f16x8 *>(reinterpret_cast<const _Float16 *>(po) + off);
    a = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    b = f32x4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
  } else {
    const bf16x8 v = *reinterpret_cast<const bf16x8 *>(reinterpret_cast<const __bf16 *>(po) + off);
    a = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    b = f32x4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
  }
}

// The same eight elements as raw bits (two 16-byte words for fp32, one for
// 16-bit elements), converted by unpack_partial8 where they are used: a
// conversion next to the load would make the wave wait for it there.
template <int PK>
__device__ __forceinline__ void load_partial8_raw(const void *po, int64_t off, i32x4 &r0, i32x4 &r1) {
  if constexpr (PK == 0) {
    const i32x4 *src = reinterpret_cast<const i32x4 *>(reinterpret_cast<const float *>(po) + off);
    r0 = src[0];
    r1 = src[1];
  } else {
    r0 = *reinterpret_cast<const i32x4 *>(reinterpret_cast<const uint16_t *>(po) + off);
    r1 = i32x4{0, 0, 0, 0};
  }
}
template <int PK>
__device__ __forceinline__ void unpack_partial8(i32x4 r0, i32x4 r1, f32x4 &a, f32x4 &b) {
  if constexpr (PK == 0) {
    a = __builtin_bit_cast(f32x4, r0);
    b = __builtin_bit_cast(f32x4, r1);
  } else if constexpr (PK == 1) {
    const f16x8 v = __builtin_bit_cast(f16x8, r0);
    a = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    b = f32x4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
  } else {
    const bf16x8 v = __builtin_bit_cast(bf16x8, r0);
    a = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    b = f32x4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
  }
}

// ---------------------------------------------------------------------------
// Single-launch path for small batches
// ---------------------------------------------------------------------------
// One workgroup of kFusedWaves waves per (sequence, KV head) pair: wave w
// streams the w-th of kFusedWaves equal token ranges of the sequence (a
// multiple of 32 tokens, at most 1024: one page-id register; blocks of 32
// fp8 tokens or 16 tokens of a 16-bit cache) through the
// partial kernel's per-unit math, NBF blocks in flight, and the waves'
// online-softmax states meet in LDS, where every thread of the workgroup folds
// them and writes output rows and LSE.  Nothing goes through the split
// workspace and no merge kernel runs: for a batch whose pairs fit the CUs at
// once this is the whole call (the host's fused_fits decides; l20_pd_single_launch
// reports it).
// Split mode (p.fused_split = the split size S): one workgroup per (split,
// sequence, KV head), wave w streaming tokens [sS + wS/8, sS + (w+1)S/8) of
// split s, the waves folded in LDS as above; a sequence of one split writes
// its output rows and LSE (and marks slot 0 final), the others write split
// s's partial (o / l, m, l) into the workspace, and the merge kernel
// finishes them.  For batches whose (split, sequence, KV head) triples fit
// the CUs at once with a few blocks per wave: the whole KV streams in one
// burst, where the persistent partial kernel keeps two blocks per wave in
// flight over longer units.
constexpr int kFusedWaves = 8;
constexpr int kFusedMaxTokens = kFusedWaves * 1024;

// Where finish_with puts a wave's normalised o row, running max and sum: the
// fold's LDS slots, [wave][column][dim] and [wave][column] (the fields
// finish_with reads, named as in PartialParams).
struct FoldSlots {
  int q_len, group, po_kind;
  float *po;
  int64_t po_srow, po_shead, po_ssplit;
  float *pm;
  int64_t pm_srow, pm_shead, pm_ssplit;
  float *pl;
  int64_t pl_srow, pl_shead, pl_ssplit;
  void *out;
  int64_t o_srow, o_shead;
  float *lse;
  int64_t lse_srow, lse_shead;
};

// NQT query tiles of 16 columns (G x q_len <= 16 NQT); TREE: ancestor-mask
// verification as in the partial kernel.  The fold slots hold fp32 rows for
// one tile and fp16 rows for two (fp32 would take 128 KB of LDS), the
// precision of the 16-bit split workspaces.
template <typename QT, int KT, int D, int NQT, bool TREE, int NBF, bool SPLIT>
__global__ __launch_bounds__(64 * kFusedWaves) void pd_fp8_fused(PartialParams p) {
  typedef KvUnit<QT, KT, D, NQT, TREE, KT != 1 && D == 128 && (NBF == 1 || NQT == 1)> U;
  constexpr int kTok = U::kTok;
  constexpr int kCols = 16 * NQT;
  typedef typename std::conditional<NQT == 1, float, _Float16>::type FT;
  typedef typename U::Block Block;
  typedef typename U::qvec8 qvec8;
  __shared__ __attribute__((aligned(16))) char s_kx[U::kKLines ? kFusedWaves * U::kKxBytes : 16];
  __shared__ __attribute__((aligned(16))) FT s_o[kFusedWaves][kCols][D];
  __shared__ float s_m[kFusedWaves][kCols], s_l[kFusedWaves][kCols];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15;
  const int j = lane >> 4;
  // split mode as a separate instance: the whole-sequence launch keeps none of
  // its arithmetic
  const int SS = SPLIT ? p.fused_split : 0;
  const unsigned int pairs = (unsigned int)p.batch * (unsigned int)p.num_kv_heads;
  const int split = SS ? (int)(blockIdx.x / pairs) : 0;
  const int pair = (int)(blockIdx.x - (unsigned int)split * pairs);
  const int b = (int)((unsigned int)pair / (unsigned int)p.num_kv_heads);
  const int kvh = pair - b * p.num_kv_heads;
  char *const kx = s_kx + (U::kKLines ? wave * U::kKxBytes : 0);
  const int q_len = p.q_len;
  // (whole sequences: the host launches this kernel only when l_cap <=
  // kFusedMaxTokens; splits: the host checks S / kFusedWaves <= 1024 and
  // the block size divides it).  The length loads first, with the kernel
  // arguments: loaded after the page list's row, it took one more scalar
  // round trip (config 1 5.80 -> 6.11 us per call, config 2 in the split mode
  // 13.56 -> 13.81).
  const int L = SS ? clamped_len(p, b) : min(clamped_len(p, b), kFusedMaxTokens);
  const int n_b = SS ? splits_of_len(L, SS) : 1;
  if (split >= n_b) return;  // the sequence has no such split (the whole workgroup)
  const int32_t *row = p.indptr ? p.bt + uniform_ld(p.indptr, b) : p.bt + (int64_t)b * p.bt_srow;
  const int npages = p.indptr ? uniform_ld(p.indptr, b + 1) - uniform_ld(p.indptr, b) : p.bt_pages;
  auto tile_id = [&](int T) {
    const int m = p.page_mult;
    if (m == 1) {
      const int e = row[T];
      return (e >= 0 && (int64_t)e < p.num_pages) ? e : -1;
    }
    const int qq = (int)__umulhi((unsigned int)T, p.page_magic);  // T / m
    const int e = row[qq];
    const int64_t v = (int64_t)e * m + (T - qq * m);
    return (e >= 0 && v < p.num_pages) ? (int)v : -1;
  };
  const int sEnd = SS ? min((split + 1) * SS, L) : L;
  // (split mode: loading the span's page ids with the length instead, before
  // it is known, measured 0.15-0.2 us slower per call)
  const int S = SS ? SS / kFusedWaves : max(32, ((L + kFusedWaves - 1) / kFusedWaves + 31) & ~31);
  const int start = split * SS + wave * S;
  const int uEnd = min(start + S, sEnd);
  const int tiles = max(0, (uEnd - start + kPage - 1) / kPage);
  const int nU = KT != 1 ? (tiles + 1) >> 1 : tiles;
  // page ids of the wave's range: lane t -> tile t (-1 past the range, past
  // the page list, and for an id outside the cache)
  int pid = -1;
  if (lane < tiles && lane < npages * p.page_mult - start / kPage) pid = tile_id(start / kPage + lane);
  qvec8 qop[NQT][U::NS];
  U::load_q(p, b, kvh, qop, n16, j);
  int tree[TREE ? NQT : 1] = {};
  U::load_tree(p, b, tree, n16);
  const float k_scale = p.k_scale_ph ? uniform_ld(p.k_scale_ph, kvh) : p.k_scale;
  const float v_scale = p.v_scale_ph ? uniform_ld(p.v_scale_ph, kvh) : p.v_scale;
  const float c_log2 = k_scale * p.qk_scale_log2;
  // masking as in the partial kernel: keys before draft0 are seen by every
  // column; draft key draft0 + j by draft row i when j <= i (causal: lim is
  // the column's last visible key) or when bit j of its ancestor word is set
  const int draft0 = L - q_len;
  int lim[TREE ? 1 : NQT] = {};
  if constexpr (!TREE) {
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) lim[qt] = min(uEnd - 1, draft0 + (16 * qt + n16) % q_len);
  }
  const int min_lim = min(uEnd - 1, TREE ? draft0 - 1 : draft0);

  U st;
  st.reset();
  // block k lives in buf[k % NBF]; every buffer loads before the loop (a
  // block past the range reads nothing: its page ids are -1)
  Block buf[NBF];
#pragma unroll
  for (int i = 0; i < NBF; ++i) U::load_block(p, buf[i], pid, kvh, i, 3, n16, j);
  // block k, then the refill of its buffer with block k + NBF: K as soon as
  // the scores have consumed r.k, V after the block (the same loads on every
  // path; past the range the page ids are -1)
  auto step = [&](Block &r, int k) {
    int pg[2] = {-1, -1};
    if (k + NBF < nU) U::block_pages(pid, k + NBF, pg);
    st.compute_block(r, pid, k, start + kTok * k, uEnd, draft0, lim, min_lim, tree, qop, c_log2, j, kx,
                     [&]() { U::load_pages(p, r, pg, kvh, 1, n16, j); });
    U::load_pages(p, r, pg, kvh, 2, n16, j);
  };
  int k = 0;
  for (; k + NBF <= nU; k += NBF) {
#pragma unroll
    for (int i = 0; i < NBF; ++i) step(buf[i], k + i);
  }
#pragma unroll
  for (int i = 0; i < NBF - 1; ++i)
    if (k + i < nU) step(buf[i], k + i);

  // every wave's (o / l, m, l) into its LDS slot: column 16 qt + n16 =
  // g * q_len + i at [wave][column]
  FoldSlots fs;
  fs.q_len = q_len;
  fs.group = p.group;
  fs.po_kind = NQT == 1 ? 0 : 1;
  fs.po = reinterpret_cast<float *>(&s_o[0][0][0]);
  fs.po_srow = D;
  fs.po_shead = (int64_t)q_len * D;
  fs.po_ssplit = kCols * D;
  fs.pm = &s_m[0][0];
  fs.pm_srow = 1;
  fs.pm_shead = q_len;
  fs.pm_ssplit = kCols;
  fs.pl = &s_l[0][0];
  fs.pl_srow = 1;
  fs.pl_shead = q_len;
  fs.pl_ssplit = kCols;
  fs.out = nullptr;
  fs.o_srow = fs.o_shead = 0;
  fs.lse = nullptr;
  fs.lse_srow = fs.lse_shead = 0;
  st.finish_with(&fs, 0, 0, false, 0, wave, false, v_scale, n16, j, kx);
  __syncthreads();

  // fold: 4 dims of one column per thread and step
  const int mcols = p.group * q_len;
  constexpr int kQ = D / 4;
  for (int idx = threadIdx.x; idx < mcols * kQ; idx += 64 * kFusedWaves) {
    const int col = idx / kQ;
    const int d0 = 4 * (idx - col * kQ);
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kFusedWaves; ++w)
      if (s_l[w][col] > 0.0f) mx = fmaxf(mx, s_m[w][col]);
    float wsum = 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kFusedWaves; ++w) {
        const float l = s_l[w][col];
        if (l > 0.0f) {
          const float e = __builtin_amdgcn_exp2f(s_m[w][col] - mx) * l;
          wsum += e;
          f32x4 o;
          if constexpr (NQT == 1) {
            o = *reinterpret_cast<const f32x4 *>(&s_o[w][col][d0]);
          } else {
            const f16x2 lo = *reinterpret_cast<const f16x2 *>(&s_o[w][col][d0]);
            const f16x2 hi = *reinterpret_cast<const f16x2 *>(&s_o[w][col][d0 + 2]);
            o = f32x4{(float)lo[0], (float)lo[1], (float)hi[0], (float)hi[1]};
          }
          acc += e * o;
        }
      }
    }
    const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
    const int g = col / q_len;
    const int i = col - g * q_len;
    const int64_t orow = (int64_t)b * q_len + i;
    const int64_t h = (int64_t)kvh * p.group + g;
    if (n_b > 1) {
      // split mode: this split's partial, in the workspace's element type
      const int64_t po_idx = orow * p.po_srow + h * p.po_shead + split * p.po_ssplit + d0;
      if (p.po_kind == 0) {
        *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.po) + po_idx) = acc * inv;
      } else {
        _Float16 *dst = reinterpret_cast<_Float16 *>(p.po) + po_idx;
        *reinterpret_cast<i32x2 *>(dst) =
            p.po_kind == 2 ? i32x2{pack2<__bf16>(acc[0] * inv, acc[1] * inv), pack2<__bf16>(acc[2] * inv, acc[3] * inv)}
                           : i32x2{pack2<_Float16>(acc[0] * inv, acc[1] * inv), pack2<_Float16>(acc[2] * inv, acc[3] * inv)};
      }
      if (d0 == 0) {
        p.pm[orow * p.pm_srow + h * p.pm_shead + split * p.pm_ssplit] = mx;
        p.pl[orow * p.pl_srow + h * p.pl_shead + split * p.pl_ssplit] = wsum;
      }
      continue;
    }
    // merge: the row is final (a sequence of one split, split mode)
    if (SS && d0 == 0 && p.num_splits > 1) p.pm[orow * p.pm_srow + h * p.pm_shead] = INFINITY;
    QT *dst = reinterpret_cast<QT *>(p.out) + orow * p.o_srow + h * p.o_shead + d0;
    *reinterpret_cast<i32x2 *>(dst) = i32x2{pack2<QT>(acc[0] * inv, acc[1] * inv), pack2<QT>(acc[2] * inv, acc[3] * inv)};
    if (d0 == 0 && p.lse)
      p.lse[orow * p.lse_srow + h * p.lse_shead] =
          wsum > 0.0f ? kLn2 * (mx + __builtin_amdgcn_logf(wsum)) : -INFINITY;  // v_log_f32 is log2
  }
}

struct MergeParams {
  const void *po;
  int64_t po_srow, po_shead, po_ssplit;
  const float *pm;
  int64_t pm_srow, pm_shead, pm_ssplit;
  const float *pl;
  int64_t pl_srow, pl_shead, pl_ssplit;
  const int32_t *seq_lens;
  void *out;
  int64_t o_srow, o_shead;
  float *lse;
  int64_t lse_srow, lse_shead;
  int q_len, split_size, num_splits, po_kind;  // po_kind as in PartialParams
  int l_cap;  // same clamp as the partial kernel
  int rows, num_q_heads;
  // Load every step of each wave's first step group before the split counts
  // are known (a small workspace: reading slots past a row's count costs
  // less than the round trip it saves).  Selects the kernel's SPEC instance.
  int spec_all;
};

// WPP waves per (query row, q head) pair (WPP = 1, 2, 4, 8 or 16: enough
// that each wave holds at most four steps of slots).  Lane l of a wave owns
// dims [8c, 8c + 8) of slot group g (c = l % (D/8), g = l / (D/8)); wave w of
// a pair takes slots (w + WPP * step) * G + g, G = 512/D groups, so every load
// of a wave is independent and issued together.  Each wave folds its groups
// with shuffles; with WPP > 1 the pair's waves then combine through LDS.
template <typename QT, int D, int WPP, int PK, bool SPEC>
__global__ __launch_bounds__(WPP > 4 ? 64 * WPP : 256) void pd_merge(MergeParams p) {
  constexpr int CH = D / 8;                // 8-dim chunks per row
  constexpr int SG = 64 / CH;              // slot groups per wave
  constexpr int WPB = WPP > 4 ? WPP : 4;   // waves per workgroup
  constexpr int PPB = WPB / WPP;           // pairs per workgroup
  __shared__ float s_m[WPB], s_w[WPB];
  __shared__ f32x4 s_acc[WPP > 1 ? WPB : 1][CH][2];
  const int lane = threadIdx.x & 63;
  // wave-uniform (SGPR): the row, its length and the step tests below are
  // scalar, so a test around a step's loads is a scalar branch, not an
  // exec-masked one that waits for every load before the next step's
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wp = wave % WPP;
  const int c = lane % CH;
  const int g = lane / CH;
  // (row, head) pairs number below 2^31 (host check): 32-bit division
  const uint32_t pair = blockIdx.x * (uint32_t)PPB + (uint32_t)(wave / WPP);
  const bool live = pair < (uint32_t)(p.rows * p.num_q_heads);
  const int row = live ? (int)(pair / (uint32_t)p.num_q_heads) : 0;
  const int h = live ? (int)(pair - (uint32_t)row * (uint32_t)p.num_q_heads) : 0;
  const float *pm = p.pm + (int64_t)row * p.pm_srow + (int64_t)h * p.pm_shead;
  const float *pl = p.pl + (int64_t)row * p.pl_srow + (int64_t)h * p.pl_shead;
  const int64_t base = (int64_t)row * p.po_srow + (int64_t)h * p.po_shead + 8 * c;
  // The first step's slot of each lane group loads before the row's split
  // count is known, in the round trip of the sequence length (slot 0 past
  // the workspace; a slot past the count is not folded): rows of at most
  // SG * WPP splits then take one round trip less.
  float m_pre, l_pre;
  i32x4 r0_pre, r1_pre;
  {
    const int s = wp * SG + g;
    const int sl = s < p.num_splits ? s : 0;
    m_pre = pm[(int64_t)sl * p.pm_ssplit];
    l_pre = pl[(int64_t)sl * p.pl_ssplit];
    load_partial8_raw<PK>(p.po, base + (int64_t)sl * p.po_ssplit, r0_pre, r1_pre);
  }
  // With SPEC (the host's spec_all), the first group's other steps load here
  // as well.
  constexpr int kSteps = 4;
  float ms_pre[kSteps], ls_pre[kSteps];
  i32x4 r0s_pre[kSteps], r1s_pre[kSteps];
  if constexpr (SPEC) {
#pragma unroll
    for (int k = 1; k < kSteps; ++k) {
      const int s = wp * SG + k * WPP * SG + g;
      const int sl = s < p.num_splits ? s : 0;
      ms_pre[k] = pm[(int64_t)sl * p.pm_ssplit];
      ls_pre[k] = pl[(int64_t)sl * p.pl_ssplit];
      load_partial8_raw<PK>(p.po, base + (int64_t)sl * p.po_ssplit, r0s_pre[k], r1s_pre[k]);
    }
  }
  int n = 0;
  if (live) {
    const int L = max(0, min(p.seq_lens[row / p.q_len], p.l_cap));
    n = (L > 0) ? (L + p.split_size - 1) / p.split_size : 0;
  }
  if (WPP == 1 && n <= 1) return;  // the partial kernel wrote this row (or the empty row) directly
  // Online merge (max, weight sum, weighted rows) over the lane's slots; NaN
  // slots (a run continued from an earlier slot) never enter the sums.
  // final_row: one run wrote the whole row already (slot 0's m is +inf).  Only
  // lanes g == 0 of wave 0 of the pair write, and their first step loads slot
  // 0, so they take it from there rather than from a load of its own (which
  // the first step's loads would wait for).
  bool final_row = false;
  float mx = -INFINITY, wsum = 0.0f;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const int n_here = n > 1 ? n : 0;
  // Steps of a wave in groups of kSteps: every load of a group is issued
  // before the group is folded (one round trip for up to kSteps steps); in a
  // step that reaches the row's count, a slot past it loads slot 0, which
  // exists whenever n > 1, and is not folded; a step wholly past it loads
  // nothing.  (Against a loop unrolled by two with the loads under the slot
  // test: call minus partial kernel 5.76 -> 5.57 us at config 3, 8.2 ->
  // 7.65 us at config 4.)
  auto fold = [&](int s, float m, float l, f32x4 a0, f32x4 a1) {
    if (s < n_here && m == m && m != -INFINITY) {
      const float m_new = fmaxf(mx, m);
      const float a_old = __builtin_amdgcn_exp2f(mx - m_new);  // 0 while mx == -inf
      const float w = __builtin_amdgcn_exp2f(m - m_new) * l;
      acc0 = acc0 * a_old + w * a0;
      acc1 = acc1 * a_old + w * a1;
      wsum = wsum * a_old + w;
      mx = m_new;
    }
  };
  for (int s0 = wp * SG; s0 < n_here; s0 += kSteps * WPP * SG) {
    // the first group's step 0 is the preload, folded from its own
    // registers (a copy would wait for it before the later steps' loads)
    const bool first = s0 == wp * SG;
    float ms[kSteps], ls[kSteps];
    i32x4 r0[kSteps], r1[kSteps];
    // the group's remaining steps load together, or (a row that the
    // preloaded step covers: a wave-uniform test) not at all
    const bool rest = !first || n_here > s0 + WPP * SG;
    if (SPEC && first) {
#pragma unroll
      for (int k = 1; k < kSteps; ++k) {
        ms[k] = ms_pre[k];
        ls[k] = ls_pre[k];
        r0[k] = r0s_pre[k];
        r1[k] = r1s_pre[k];
      }
    } else if (rest) {
#pragma unroll
      for (int k = 0; k < kSteps; ++k) {
        if (k == 0 && first) continue;
        const int s = s0 + k * WPP * SG + g;
        const int sl = s < n_here ? s : 0;
        ms[k] = pm[(int64_t)sl * p.pm_ssplit];
        ls[k] = pl[(int64_t)sl * p.pl_ssplit];
        load_partial8_raw<PK>(p.po, base + (int64_t)sl * p.po_ssplit, r0[k], r1[k]);
      }
    }
    if (first) {
      if (s0 == 0 && m_pre == INFINITY) final_row = true;
      f32x4 a0, a1;
      unpack_partial8<PK>(r0_pre, r1_pre, a0, a1);
      fold(s0 + g, m_pre, l_pre, a0, a1);
    }
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      if ((k == 0 && first) || !rest) continue;
      f32x4 a0, a1;
      unpack_partial8<PK>(r0[k], r1[k], a0, a1);
      fold(s0 + k * WPP * SG + g, ms[k], ls[k], a0, a1);
    }
  }
  // LSE-combine (mx, wsum, acc) with another partial state.
  auto combine = [&](float m_o, float w_o, f32x4 a0_o, f32x4 a1_o) {
    const float m_new = fmaxf(mx, m_o);
    const float ms = (m_new == -INFINITY) ? 0.0f : m_new;
    const float a = __builtin_amdgcn_exp2f(mx - ms);
    const float bo = __builtin_amdgcn_exp2f(m_o - ms);
    acc0 = acc0 * a + a0_o * bo;
    acc1 = acc1 * a + a1_o * bo;
    wsum = wsum * a + w_o * bo;
    mx = m_new;
  };
  // fold the slot groups (lane bits at and above log2(CH))
#pragma unroll
  for (int off = CH; off < 64; off <<= 1) {
    f32x4 a0_o, a1_o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a0_o[e] = __shfl_xor(acc0[e], off);
      a1_o[e] = __shfl_xor(acc1[e], off);
    }
    combine(__shfl_xor(mx, off), __shfl_xor(wsum, off), a0_o, a1_o);
  }
  if constexpr (WPP > 1) {
    // fold the pair's waves: every wave publishes its state, the first folds
    if (g == 0) {
      s_acc[wave][c][0] = acc0;
      s_acc[wave][c][1] = acc1;
      if (c == 0) {
        s_m[wave] = mx;
        s_w[wave] = wsum;
      }
    }
    __syncthreads();
    if (wp != 0 || n <= 1) return;
#pragma unroll
    for (int k = 1; k < WPP; ++k)
      combine(s_m[wave + k], s_w[wave + k], s_acc[wave + k][c][0], s_acc[wave + k][c][1]);
  }
  const float msafe = (mx == -INFINITY) ? 0.0f : mx;
  if (final_row) return;
  if (g != 0) return;
  const float inv = (wsum > 0.0f) ? 1.0f / wsum : 0.0f;
  QT *dst = reinterpret_cast<QT *>(p.out) + (int64_t)row * p.o_srow + (int64_t)h * p.o_shead + 8 * c;
  const i32x4 w = {pack2<QT>(acc0[0] * inv, acc0[1] * inv), pack2<QT>(acc0[2] * inv, acc0[3] * inv),
                   pack2<QT>(acc1[0] * inv, acc1[1] * inv), pack2<QT>(acc1[2] * inv, acc1[3] * inv)};
  *reinterpret_cast<i32x4 *>(dst) = w;
  if (c == 0 && p.lse) {
    p.lse[(int64_t)row * p.lse_srow + (int64_t)h * p.lse_shead] =
        (wsum > 0.0f) ? kLn2 * (msafe + __builtin_amdgcn_logf(wsum)) : -INFINITY;
  }
}

// Narrow merge for at most kNarrowSlots split slots: lane l owns dims
// [8c, 8c + 8) of one (query row, q head) pair (c = l % (D/8); 64 / (D/8)
// pairs per wave) across every slot of it, so the fold needs no shuffles.
// NSL (2, 4 or 8) slots are read in the round trip that fetches the sequence
// length, with no branch around any load: a slot at or past num_splits reads
// slot 0 again (NSL is the smallest of the three >= num_splits), and slots at
// or past the row's split count hold whatever an earlier call left and are
// not folded.
constexpr int kNarrowSlots = 8;
template <typename QT, int D, int PK, int NSL>
__global__ __launch_bounds__(256) void pd_merge_narrow(MergeParams p) {
  constexpr int CH = D / 8;     // 8-dim chunks per row
  constexpr int PPW = 64 / CH;  // pairs per wave
  static_assert(NSL <= kNarrowSlots, "narrow merge slots");
  const int lane = threadIdx.x & 63;
  const int c = lane % CH;
  // (row, head) pairs number below 2^31 (host check): 32-bit division
  const uint32_t pair = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * PPW + lane / CH;
  if (pair >= (uint32_t)(p.rows * p.num_q_heads)) return;
  const int row = (int)(pair / (uint32_t)p.num_q_heads);
  const int h = (int)(pair - (uint32_t)row * (uint32_t)p.num_q_heads);
  const float *pm = p.pm + (int64_t)row * p.pm_srow + (int64_t)h * p.pm_shead;
  const float *pl = p.pl + (int64_t)row * p.pl_srow + (int64_t)h * p.pl_shead;
  const int64_t base = (int64_t)row * p.po_srow + (int64_t)h * p.po_shead + 8 * c;
  float ms[NSL], ls[NSL];
  f32x4 o0[NSL], o1[NSL];
#pragma unroll
  for (int s = 0; s < NSL; ++s) {
    const int sl = s < p.num_splits ? s : 0;
    ms[s] = pm[(int64_t)sl * p.pm_ssplit];
    ls[s] = pl[(int64_t)sl * p.pl_ssplit];
    load_partial8<PK>(p.po, base + (int64_t)sl * p.po_ssplit, o0[s], o1[s]);
  }
  const int L = max(0, min(p.seq_lens[row / p.q_len], p.l_cap));
  const int n = (L > 0) ? (L + p.split_size - 1) / p.split_size : 0;
  if (n <= 1) return;                // the partial kernel wrote this row (or the empty row) directly
  if (ms[0] == INFINITY) return;     // ... or marked it final
  float mx = -INFINITY, wsum = 0.0f;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NSL; ++s) {
    if (s < n && ms[s] == ms[s] && ms[s] != -INFINITY) {
      const float m_new = fmaxf(mx, ms[s]);
      const float a_old = __builtin_amdgcn_exp2f(mx - m_new);  // 0 while mx == -inf
      const float w = __builtin_amdgcn_exp2f(ms[s] - m_new) * ls[s];
      acc0 = acc0 * a_old + w * o0[s];
      acc1 = acc1 * a_old + w * o1[s];
      wsum = wsum * a_old + w;
      mx = m_new;
    }
  }
  const float inv = (wsum > 0.0f) ? 1.0f / wsum : 0.0f;
  QT *dst = reinterpret_cast<QT *>(p.out) + (int64_t)row * p.o_srow + (int64_t)h * p.o_shead + 8 * c;
  *reinterpret_cast<i32x4 *>(dst) = i32x4{pack2<QT>(acc0[0] * inv, acc0[1] * inv), pack2<QT>(acc0[2] * inv, acc0[3] * inv),
                                          pack2<QT>(acc1[0] * inv, acc1[1] * inv), pack2<QT>(acc1[2] * inv, acc1[3] * inv)};
  if (c == 0 && p.lse) {
    const float msafe = (mx == -INFINITY) ? 0.0f : mx;
    p.lse[(int64_t)row * p.lse_srow + (int64_t)h * p.lse_shead] =
        (wsum > 0.0f) ? kLn2 * (msafe + __builtin_amdgcn_logf(wsum)) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Bulk dequantisers (same conversions as the attention kernel)
// ---------------------------------------------------------------------------
// Four consecutive codes starting at i as one dword (zero-filled past n).
__device__ __forceinline__ int load_codes4(const uint8_t *src, int64_t i, int64_t n) {
  if (i + 4 <= n && ((reinterpret_cast<uintptr_t>(src) + i) & 3) == 0)
    return *reinterpret_cast<const int *>(src + i);
  int w = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i + e < n) w |= (int)src[i + e] << (8 * e);
  return w;
}

__global__ void dequant_f32_kernel(const uint8_t *src, float *dst, int64_t n, float scale) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  const int w = load_codes4(src, i, n);
  const f32x2 lo = fp8x2_f32<false>(w, false);
  const f32x2 hi = fp8x2_f32<false>(w, true);
  const float v[4] = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i + e < n) dst[i + e] = v[e] * scale;
}

__global__ void dequant_bf16_kernel(const uint8_t *src, uint16_t *dst, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  const int w = load_codes4(src, i, n);
  // Same conversion as the attention kernel's K operand; words, not lanes.
  const i32x4 both = __builtin_bit_cast(i32x4, fp8x8_to<bf16x8, false>(w, 0));
  const uint32_t lo = (uint32_t)both[0];
  const uint32_t hi = (uint32_t)both[1];
  if (i + 4 <= n && ((reinterpret_cast<uintptr_t>(dst + i) & 7) == 0)) {
    *reinterpret_cast<i32x2 *>(dst + i) = i32x2{(int)lo, (int)hi};
    return;
  }
  const uint32_t words[2] = {lo, hi};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i + e < n) dst[i + e] = (uint16_t)(words[e >> 1] >> (16 * (e & 1)));
}

// ---------------------------------------------------------------------------
// HBM calibration kernels: a pure streaming read and a plain copy, used to
// measure the read ceiling of the device and to scale FETCH_SIZE/WRITE_SIZE.
// ---------------------------------------------------------------------------
// Workgroup i reads the i-th contiguous chunk of `chunk` bytes through a
// buffer resource, 16 loads of 16 bytes per lane in flight (contiguous
// chunks stream faster than a grid-stride walk: 6.2-6.3 vs 5.5-6.0 TB/s on
// MI355X over 1 GiB buffers).  Loads past the chunk return zero (range check).
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t *src, int64_t nbytes, int64_t chunk,
                                                         int *sink) {
  constexpr int U = 16;
  constexpr int kStep = 256 * 16;  // bytes one load instruction of the workgroup covers
  const int64_t base = (int64_t)blockIdx.x * chunk;
  if (base >= nbytes) return;
  const int len = (int)(nbytes - base < chunk ? nbytes - base : chunk);
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src) + base, (short)0, len, kBufferWord3);
  int acc = 0;
  for (int off = (int)threadIdx.x * 16; off < len; off += U * kStep) {
    i32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      v[u] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + u * kStep, 0, kStreamPolicy));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x7fffffff) sink[blockIdx.x] = acc;  // keeps the loads live; practically never stores
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const i32x4 *src, i32x4 *dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace l20pd

// ===========================================================================
// Host side: validation, launch, C ABI
// ===========================================================================
namespace {

thread_local char g_last_error[512] = "";

int32_t fail(int32_t code, const char *msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return code;
}

int32_t check_args(const l20_pd_fp8_args *a) {
  if (!a) return fail(L20_PD_EINVAL, "null argument block");
  if (a->query_dtype != L20_PD_BF16 && a->query_dtype != L20_PD_FP16)
    return fail(L20_PD_EINVAL, "query must be bf16 or fp16");
  if (a->kv_dtype != L20_PD_KV_FP8_E4M3 && a->kv_dtype != L20_PD_KV_FP16 && a->kv_dtype != L20_PD_KV_BF16 &&
      a->kv_dtype != L20_PD_KV_FP8_E5M2)
    return fail(L20_PD_EINVAL, "unknown K/V cache dtype");
  const bool kv16 = a->kv_dtype == L20_PD_KV_FP16 || a->kv_dtype == L20_PD_KV_BF16;
  if (kv16 && (a->kv_dtype == L20_PD_KV_BF16) != (a->query_dtype == L20_PD_BF16))
    return fail(L20_PD_EINVAL, "query and 16-bit K/V cache must have the same dtype");
  const int64_t es = kv16 ? 2 : 1;  // bytes per cache element
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(L20_PD_EINVAL, "NHD cache only: head_dim must be 64 or 128");
  // Pages of any multiple of 16 tokens (the reference's vLLM hook passes its
  // block size through, integrations/vllm/l20_paged_split_kv.py:156,182-200).
  if (a->page_size < 16 || a->page_size % 16 != 0 || a->page_size > 4096)
    return fail(L20_PD_EINVAL, "NHD cache only: page_size must be a multiple of 16 from 16 through 4096");
  if (a->num_kv_heads <= 0 || a->num_q_heads <= 0)
    return fail(L20_PD_EINVAL, "head counts must be positive");
  if (a->num_q_heads % a->num_kv_heads != 0)
    return fail(L20_PD_EINVAL, "Q heads must be divisible by KV heads");
  if (a->q_len < 1) return fail(L20_PD_EINVAL, "q_len must be >= 1");
  if ((a->num_q_heads / a->num_kv_heads) * a->q_len > 32)
    return fail(L20_PD_EINVAL, "GQA group x q_len must be at most 32");
  if (a->split_size < 64 || a->split_size > 1024 || a->split_size % 16 != 0)
    return fail(L20_PD_EINVAL, "split_size must be a multiple of 16 from 64 through 1024");
  if (a->batch < 0 || a->max_seq_len < 0) return fail(L20_PD_EINVAL, "batch and max_seq_len must be >= 0");
  if (a->batch > 65535 || l20_pd_num_splits(a->max_seq_len, a->split_size) > 65535)
    return fail(L20_PD_EINVAL, "batch and the split count must be at most 65535");
  if ((int64_t)a->batch * a->q_len * a->num_q_heads > INT32_MAX)
    return fail(L20_PD_EINVAL, "batch x q_len x Q heads must be below 2^31");
  if (a->batch == 0) return L20_PD_OK;
  if (!a->query || !a->key_cache || !a->value_cache || !a->block_table || !a->seq_lens || !a->output)
    return fail(L20_PD_EINVAL, "null tensor pointer");
  if (((uintptr_t)a->page_indptr % 4) != 0) return fail(L20_PD_EINVAL, "page_indptr must be int32-aligned");
  if (((uintptr_t)a->tree_mask % 4) != 0 || a->tree_mask_stride_batch < 0)
    return fail(L20_PD_EINVAL, "tree_mask must be int32 [batch, q_len] (batch stride >= 0)");
  if (a->num_pages <= 0) return fail(L20_PD_EINVAL, "K/V cache has no pages");
  if (a->page_size > 16) {
    // read as 16-token sub-pages: a page's tokens must be contiguous
    if (a->k_stride_page != a->page_size * a->k_stride_token || a->v_stride_page != a->page_size * a->v_stride_token)
      return fail(L20_PD_EINVAL, "pages of more than 16 tokens must hold them contiguously (stride_page = page_size x stride_token)");
    if (a->num_pages * (a->page_size / 16) > INT32_MAX || (int64_t)a->bt_max_pages * a->page_size > INT32_MAX)
      return fail(L20_PD_EINVAL, "K/V cache and block table must hold fewer than 2^35 tokens");
    // the kernels divide 16-token tile indices by page_size / 16 through a reciprocal
    if ((int64_t)a->max_seq_len / 16 + 128 >= (((int64_t)1 << 32) / (a->page_size / 16)))
      return fail(L20_PD_EINVAL, "max_seq_len is too long for this page_size");
  }
  const int32_t n_s = l20_pd_num_splits(a->max_seq_len, a->split_size);
  if (n_s > 1) {
    if (!a->partial_output || !a->partial_max || !a->partial_sum)
      return fail(L20_PD_EINVAL, "partial output workspace has wrong shape");
    if (a->partial_splits < n_s) return fail(L20_PD_EINVAL, "partial output workspace has wrong shape");
    if (a->partial_dtype != L20_PD_FP32 && a->partial_dtype != L20_PD_FP16 && a->partial_dtype != L20_PD_BF16)
      return fail(L20_PD_EINVAL, "partial output must be fp32, fp16 or bf16");
  }
  for (int which = 0; which < 2; ++which) {
    const int64_t st = which ? a->v_stride_token : a->k_stride_token;
    const int64_t sh = which ? a->v_stride_head : a->k_stride_head;
    if (st < 0 || sh < 0 || (15 * st + (int64_t)(a->num_kv_heads - 1) * sh + a->head_dim) * es > INT32_MAX)
      return fail(L20_PD_EINVAL, "K/V token and head strides must be non-negative and span less than 2 GiB per page");
  }
  if (!a->page_indptr && a->bt_max_pages * (int64_t)a->page_size < a->max_seq_len)
    return fail(L20_PD_EINVAL, "block table has fewer pages than max_seq_len needs");
  // Vector-load alignment: 16 B K chunks, V chunks of head_dim/16 elements, 16 B query chunks.
  const uint64_t kbits = (uint64_t)(uintptr_t)a->key_cache | (uint64_t)(a->k_stride_page * es) |
                         (uint64_t)(a->k_stride_token * es) | (uint64_t)(a->k_stride_head * es);
  if (kbits % 16 != 0) return fail(L20_PD_EINVAL, "K cache pointer and strides must be 16-byte aligned");
  const uint64_t vbits = (uint64_t)(uintptr_t)a->value_cache | (uint64_t)(a->v_stride_page * es) |
                         (uint64_t)(a->v_stride_token * es) | (uint64_t)(a->v_stride_head * es);
  if (vbits % (uint64_t)((a->head_dim / 16) * es) != 0)
    return fail(L20_PD_EINVAL, "V cache pointer and strides must be aligned to head_dim/16 elements");
  if (((uintptr_t)a->query % 16) != 0 || (a->q_stride_row % 8) != 0 || (a->q_stride_head % 8) != 0)
    return fail(L20_PD_EINVAL, "query pointer and strides must be 16-byte aligned");
  if (((uintptr_t)a->output % 16) != 0 || (a->o_stride_row % 8) != 0 || (a->o_stride_head % 8) != 0)
    return fail(L20_PD_EINVAL, "output pointer and strides must be 16-byte aligned");
  if (n_s > 1 && a->partial_dtype != L20_PD_FP32 &&
      (((uintptr_t)a->partial_output % 16) != 0 || a->po_stride_row % 8 || a->po_stride_head % 8 ||
       a->po_stride_split % 8))
    return fail(L20_PD_EINVAL, "16-bit partial output must be 16-byte aligned");
  if (n_s > 1 && a->partial_dtype == L20_PD_FP32 &&
      (((uintptr_t)a->partial_output % 16) != 0 || a->po_stride_row % 4 || a->po_stride_head % 4 ||
       a->po_stride_split % 4))
    return fail(L20_PD_EINVAL, "fp32 partial output must be 16-byte aligned");
  return L20_PD_OK;
}

// Waves per partial workgroup: the largest divisor of the KV head count
// that is at most kMaxWaves, so every wave owns the same number of heads.
int partial_waves(int num_kv_heads) {
  for (int w = std::min(num_kv_heads, l20pd::kMaxWaves); w > 1; --w)
    if (num_kv_heads % w == 0) return w;
  return 1;
}

// Compact item numbering needs the batch's prefix in LDS.
bool partial_compact(int batch) { return batch <= l20pd::kMaxCompactBatch; }

// Workgroups the persistent partial kernel launches: enough to fill every CU
// at the kernel's occupancy, never more than there are split-major slots.
// L20_PD_MAX_WORKGROUPS (a positive integer) caps the count, which lets tests
// drive many items through each workgroup.
template <typename QT, int KT, int D, int NQT, bool TREE, int NB>
int partial_grid(int threads, size_t lds, int64_t max_items) {
  static thread_local int cached_dev = -1, cached_threads = -1, cached_blocks = 0;  // per instantiation
  static thread_local size_t cached_lds = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev != cached_dev || threads != cached_threads || lds != cached_lds) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, l20pd::pd_fp8_partial<QT, KT, D, NQT, TREE, NB>, threads,
                                                     lds) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    cached_dev = dev;
    cached_threads = threads;
    cached_lds = lds;
    cached_blocks = cus * per_cu;
  }
  int64_t blocks = cached_blocks;
  if (const char *cap = getenv("L20_PD_MAX_WORKGROUPS")) {
    const long v = strtol(cap, nullptr, 10);
    if (v > 0) blocks = std::min<int64_t>(blocks, v);
  }
  return (int)std::max<int64_t>(1, std::min<int64_t>(blocks, max_items));
}

// Two items per workgroup: instances with one query tile, two blocks in
// flight and the whole-line K pass, one KV head per wave, at most 8 waves per
// workgroup, and a launch whose persistent grid covers every split-major
// slot (every item known from the workgroup index, none numbered through
// the LDS prefix).  Config 2's shape (32 x 2048 tokens, 2 KV heads, 128-token
// splits: 512 items) then runs 256 workgroups of 4 waves instead of 512 of 2:
// 16.5-17.0 -> 15.6 us per call, fp16 partials.  With prefix-numbered items
// (config 3) the two groups of a workgroup start their first units ~6 us
// apart either way and pairing measured 0.5-3 us slower (timelines per
// wave: the second item's length prefix, decode and page ids are three
// dependent loads behind the first item's K/V burst).  L20_PD_PAIRED=0/1
// overrides the choice (measurement).
template <typename QT, int KT, int D, int NQT, bool TREE, int NB>
bool partial_paired(int num_kv_heads, int nwaves, int batch, int num_splits) {
  constexpr bool pairable = KT != 1 && D == 128 && NQT == 1 && NB == 2 && !TREE;
  if (!pairable || nwaves != num_kv_heads || 2 * nwaves > l20pd::kMaxWaves) return false;
  if (const char *env = getenv("L20_PD_PAIRED")) return env[0] == '1';
  // The paired grid (CUs workgroups of 2 x nwaves waves at occupancy 2 waves
  // per SIMD) covers every split-major slot: no queue, no prefix.
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int64_t vslots = (int64_t)cus * (8 / nwaves);  // two virtual workgroups per workgroup
  return (int64_t)batch * num_splits <= vslots;
}

template <typename QT, int KT, int D, int NQT, bool TREE, int NB>
hipError_t launch_partial(l20pd::PartialParams pp, int batch, int num_kv_heads, hipStream_t stream) {
  const int nwaves = partial_waves(num_kv_heads);
  pp.compact = partial_compact(batch) ? 1 : 0;
  pp.paired = partial_paired<QT, KT, D, NQT, TREE, NB>(num_kv_heads, nwaves, batch, pp.num_splits) ? 1 : 0;
  const int threads = 64 * nwaves * (pp.paired ? 2 : 1);
  const size_t lds = pp.compact ? (size_t)(2 * batch + 2) * sizeof(int) : 0;
  const int64_t max_items = (int64_t)batch * pp.num_splits;
  // paired: each workgroup runs two virtual workgroups of the schedule
  const int grid = partial_grid<QT, KT, D, NQT, TREE, NB>(threads, lds, pp.paired ? (max_items + 1) / 2 : max_items);
  hipLaunchKernelGGL((l20pd::pd_fp8_partial<QT, KT, D, NQT, TREE, NB>), dim3(grid), dim3(threads), lds, stream, pp);
  return hipGetLastError();
}

template <typename QT, int KT, bool TREE>
hipError_t launch_partial_mask(const l20pd::PartialParams &pp, int head_dim, int nqt, int batch, int num_kv_heads,
                               hipStream_t stream) {
  if (head_dim == 128) {
    // Units of up to 32 fp8 blocks (splits >= 1024): one block in flight per
    // wave halves the bytes queued in the memory system at full bandwidth
    // (verify shape 130.7 -> 126.4 us per call, long context 106.1 -> 104.5);
    // shorter units keep two for the latency-bound end of the launch.
    if constexpr (KT != 1)
      if (pp.split_size >= 1024)
        return nqt == 1 ? launch_partial<QT, KT, 128, 1, TREE, 1>(pp, batch, num_kv_heads, stream)
                        : launch_partial<QT, KT, 128, 2, TREE, 1>(pp, batch, num_kv_heads, stream);
    return nqt == 1 ? launch_partial<QT, KT, 128, 1, TREE, 2>(pp, batch, num_kv_heads, stream)
                    : launch_partial<QT, KT, 128, 2, TREE, 2>(pp, batch, num_kv_heads, stream);
  }
  return nqt == 1 ? launch_partial<QT, KT, 64, 1, TREE, 2>(pp, batch, num_kv_heads, stream)
                  : launch_partial<QT, KT, 64, 2, TREE, 2>(pp, batch, num_kv_heads, stream);
}

template <typename QT, int KT>
hipError_t launch_partial_shape(const l20pd::PartialParams &pp, int head_dim, int nqt, int batch, int num_kv_heads,
                                hipStream_t stream) {
  return pp.tree ? launch_partial_mask<QT, KT, true>(pp, head_dim, nqt, batch, num_kv_heads, stream)
                 : launch_partial_mask<QT, KT, false>(pp, head_dim, nqt, batch, num_kv_heads, stream);
}

// The single-launch kernel: one workgroup per (sequence, KV head), two blocks
// in flight per wave.  (Three or four blocks spill at head_dim 128 -- 256
// VGPRs and 44 / 284 bytes of scratch per lane -- and were slower on every
// shape measured: config 1 5.81 / 5.83 / 6.05 us, 128 x 1024 tokens 15.2 /
// 17.8 / 26.3 us for two / three / four.)
constexpr int kFusedNB = 2;
// Two query tiles (verification: G x q_len up to 32) keep one block in
// flight: two blocks (228 VGPRs, non-line K) measured slower on every
// verify shape (64 Q / 8 KV heads, q_len 4: 4 x 1024 tokens 16.0 against
// 18.9 us, 16 x 512 13.0 against 14.6).
constexpr int kFusedNB2 = 1;
template <typename QT, int KT, int NQT, bool TREE>
hipError_t launch_fused_tiles(const l20pd::PartialParams &pp, int head_dim, int batch, int num_kv_heads,
                              hipStream_t stream) {
  // split mode: one workgroup per (split, sequence, KV head), split-major
  const dim3 grid((unsigned)((int64_t)batch * num_kv_heads * (pp.fused_split ? pp.num_splits : 1))),
      block(64 * l20pd::kFusedWaves);
  constexpr int NB = NQT == 1 ? kFusedNB : kFusedNB2;
  if (pp.fused_split) {
    if (head_dim == 128) hipLaunchKernelGGL((l20pd::pd_fp8_fused<QT, KT, 128, NQT, TREE, NB, true>), grid, block, 0, stream, pp);
    else hipLaunchKernelGGL((l20pd::pd_fp8_fused<QT, KT, 64, NQT, TREE, NB, true>), grid, block, 0, stream, pp);
  } else {
    if (head_dim == 128) hipLaunchKernelGGL((l20pd::pd_fp8_fused<QT, KT, 128, NQT, TREE, NB, false>), grid, block, 0, stream, pp);
    else hipLaunchKernelGGL((l20pd::pd_fp8_fused<QT, KT, 64, NQT, TREE, NB, false>), grid, block, 0, stream, pp);
  }
  return hipGetLastError();
}
template <typename QT, int KT>
hipError_t launch_fused(const l20pd::PartialParams &pp, int head_dim, int nqt, int batch, int num_kv_heads,
                        hipStream_t stream) {
  if (nqt == 1)
    return pp.tree ? launch_fused_tiles<QT, KT, 1, true>(pp, head_dim, batch, num_kv_heads, stream)
                   : launch_fused_tiles<QT, KT, 1, false>(pp, head_dim, batch, num_kv_heads, stream);
  return pp.tree ? launch_fused_tiles<QT, KT, 2, true>(pp, head_dim, batch, num_kv_heads, stream)
                 : launch_fused_tiles<QT, KT, 2, false>(pp, head_dim, batch, num_kv_heads, stream);
}

// Whether a call runs as the single launch (one or two query tiles, causal
// draft rows or a tree mask): at most one (sequence, KV head) pair per CU and
// at most
// 1024 tokens per sequence the call may touch for fp8 caches (four blocks of
// 32 tokens per wave), 640 for 16-bit ones (five blocks of 16 tokens, 8 KB
// each as for fp8; 16-bit caches, 8 KV heads, per call: 4 x 512 tokens 16.1
// -> 12.8 us, 32 x 512 19.2 -> 15.6, 4 x 640 16.3 -> 14.8, 1 x 2048 16.6
// against 36.1).  Verification (64 Q / 8 KV heads, q_len 4, per call): 16 x
// 512 tokens 20.7 -> 13.0 us, 4 x 1024 19.0 -> 16.0, 8 x 1024 with 32 Q / 4
// KV heads 15.7 either way.
// Then every pair streams at once on its own CU and the split workspace and
// the merge launch are skipped.  Measured in one process against the split
// kernels (per call): config 1 10.0 -> 5.8 us, 64 x 1024 tokens (2 KV heads)
// 14.4 -> 12.2, 128 x 1024 20.4 -> 15.2; with eight blocks per wave and more
// the pairs' CUs are latency-bound (each holds 8 waves x 2 blocks x 8 KB in
// flight) and the split kernels win: config 2 (32 x 2048) 14.8 against 17.3,
// 16 x 2048 13.0 against 16.8, 32 x 4096 19.3 against 28.4.
// L20_PD_FUSED=0/1 overrides the size rule (tests and measurement; the shape
// conditions and kFusedMaxTokens always hold).
bool fused_fits(const l20_pd_fp8_args &a, const l20pd::PartialParams &pp, int nqt, bool kv16) {
  if (nqt > 2) return false;  // (the checks already limit G x q_len to 32)
  if (pp.l_cap > l20pd::kFusedMaxTokens) return false;
  if (const char *env = getenv("L20_PD_FUSED")) return env[0] == '1';
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return (int64_t)a.batch * a.num_kv_heads <= cus && pp.l_cap <= (kv16 ? 640 : 1024);
}

// The split mode's size rule (see fused_split_fits): every triple on a CU of
// its own, and at 512 (1024) tokens at least (more than) half of the CUs
// busy; at 256 tokens (one fp8 block per wave) any count.
bool split_mode_fills(int split, int64_t triples, int64_t cus) {
  if (triples > cus) return false;
  if (split == 256) return true;
  if (split == 512) return 2 * triples >= cus;
  return split == 1024 && 2 * triples > cus;
}

// Whether the partial stage of a split call runs as the single-launch kernel's
// split mode (one workgroup per (split, sequence, KV head), its waves' states
// folded in LDS, the split's partial written for the merge) rather than the
// persistent partial kernel: each wave's share of a split (S / 8 tokens) must
// be whole blocks and fit one page-id register, and by the size rule the
// split is 256, 512 or 1024 tokens (one, two or four fp8 blocks per wave, at
// most two in flight) and the (split, sequence, KV head) triples do not
// exceed the CUs and, at 512 (1024) tokens, fill at least (more than) half of
// them: one 8-wave workgroup per CU, every wave's blocks streaming at once.
// Measured in one process against the persistent kernel at the library's
// split, 33.5 MB of KV per call, µs per call: 32 x 2048 tokens, 2 KV heads
// (config 2) 13.5-13.9 against 14.7; 16 x 2048, 4 KV heads 14.1 against
// 17.6; 8 x 4096, 4 KV heads 13.9 against 17.7; 4 x 4096, 8 KV heads 14.2
// against 17.4; 1 x 16384, 8 KV heads 14.7 against 18.2; verification
// (4 x 4096, 64 / 8 heads, q_len 4) 19.9 against 24.5.  With twice the
// triples (64 x 2048, 2 KV heads: two rounds) 23.8 against 19.5, and with
// 256 or 1024-token splits at config 2 17.4 and 15.3.  At 1024-token splits,
// 67 MB of KV per call: 16 x 8192 tokens, 2 KV heads 18.4 against 19.6;
// 2 x 16384, 8 KV heads 19.6 against 23.5; 4 x 8192, 8 KV heads 19.4
// against 23.4; 8 x 8192, 4 KV heads 18.6 against 23.5; 64 x 2048, 2 KV heads
// 18.5 against 19.2.  Outside the rule it loses: 1024 triples at 1024 tokens
// (128 x 1536, 4 KV heads) 50.2 against 41.6, (2 x 65536, 8 KV heads) 62.1
// against 57.0.  At 256-token splits, 16.8 MB per call: 16 x 2048 tokens, 2 KV
// heads 10.9 against 12.9 (split 64); 8 x 2048, 4 KV heads 11.0 against 14.9;
// 4 x 2048, 8 KV heads 10.8 against 14.6; 2 x 4096, 8 KV heads 11.0 against
// 14.7.  At half the CUs (128 triples): 8 x 2048 tokens, 2 KV heads, 256-token
// splits 10.5 against 12.1 (split 64); 2 x 2048, 8 KV heads 10.1 against 14.2;
// 16 x 4096, 2 KV heads, 512-token splits 14.1 against 14.9; but config 2 at
// 1024-token splits 15.3 against 14.7.  At 256-token splits with few triples:
// 1 x 1100 tokens, 2 KV heads (10 triples) 9.6 against 11.7 (split 64);
// 3 x 2048, 2 KV heads (48) 10.3 against 11.9; 1 x 4096, 2 KV heads (32) 10.2
// against 12.0; 1 x 2048, 8 KV heads (64) 9.9 against 14.1; verification (q_len
// 4, two query tiles) 2 x 1500, 16 / 2 heads 13.4 against 12.9 (split 64;
// 19.1 at 256), 4 x 2048, 32 / 4 heads 14.0 against 16.1, 1 x 4096, 64 / 8
// heads 14.3 against 19.6.  L20_PD_FUSED_SPLIT=0/1 overrides the size rule.
bool fused_split_fits(const l20_pd_fp8_args &a, const l20pd::PartialParams &pp, int nqt, bool kv16) {
  if (nqt > 2 || pp.num_splits < 2) return false;
  const int blk = kv16 ? 16 : 32;
  if (a.split_size % (l20pd::kFusedWaves * blk) != 0 || a.split_size / l20pd::kFusedWaves > 1024) return false;
  // one workgroup per triple: the grid's x dimension bounds them (forced calls included)
  const int64_t triples = (int64_t)a.batch * a.num_kv_heads * pp.num_splits;
  if (triples >= ((int64_t)1 << 31)) return false;
  if (const char *env = getenv("L20_PD_FUSED_SPLIT")) return env[0] == '1';
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return split_mode_fills(a.split_size, triples, cus);
}

template <typename QT, int D, int WPP>
hipError_t launch_merge_wpp(const l20pd::MergeParams &mp, int64_t pairs, hipStream_t stream) {
  constexpr int WPB = WPP > 4 ? WPP : 4;
  constexpr int PPB = WPB / WPP;
  const dim3 grid((unsigned)((pairs + PPB - 1) / PPB)), block(64 * WPB);
  // separate instances: a runtime test of spec_all cost 0.06 us per call at
  // config 1, which never takes it
  if (mp.spec_all) {
    if (mp.po_kind == 0) hipLaunchKernelGGL((l20pd::pd_merge<QT, D, WPP, 0, true>), grid, block, 0, stream, mp);
    else if (mp.po_kind == 1) hipLaunchKernelGGL((l20pd::pd_merge<QT, D, WPP, 1, true>), grid, block, 0, stream, mp);
    else hipLaunchKernelGGL((l20pd::pd_merge<QT, D, WPP, 2, true>), grid, block, 0, stream, mp);
  } else {
    if (mp.po_kind == 0) hipLaunchKernelGGL((l20pd::pd_merge<QT, D, WPP, 0, false>), grid, block, 0, stream, mp);
    else if (mp.po_kind == 1) hipLaunchKernelGGL((l20pd::pd_merge<QT, D, WPP, 1, false>), grid, block, 0, stream, mp);
    else hipLaunchKernelGGL((l20pd::pd_merge<QT, D, WPP, 2, false>), grid, block, 0, stream, mp);
  }
  return hipGetLastError();
}

template <typename QT, int D, int PK, int NSL>
hipError_t launch_merge_narrow(const l20pd::MergeParams &mp, int64_t pairs, hipStream_t stream) {
  constexpr int64_t per_block = 4 * (64 / (D / 8));  // 4 waves of 64 / (D/8) pairs
  hipLaunchKernelGGL((l20pd::pd_merge_narrow<QT, D, PK, NSL>), dim3((unsigned)((pairs + per_block - 1) / per_block)),
                     dim3(256), 0, stream, mp);
  return hipGetLastError();
}

// Waves per (row, head) pair: each wave takes at most four steps of 512/D
// slots (a second wave costs more than it saves below that: config 3 with 16
// slots merged in 6.4 us on two waves per pair, 5.3 us on one).
int merge_waves_per_pair(int num_splits, int head_dim) {
  const int per_wave = 4 * (512 / head_dim);
  int w = 1;
  while (w < 16 && w * per_wave < num_splits) w <<= 1;
  return w;
}

template <typename QT, int D>
hipError_t launch_merge(const l20pd::MergeParams &mp, int rows, int heads, hipStream_t stream) {
  const int64_t pairs = (int64_t)rows * heads;
  if (mp.num_splits <= l20pd::kNarrowSlots && pairs >= 4096) {
    // a few slots and many pairs (a bandwidth-heavy merge: verify shape 10.0 ->
    // 7.4 us between the partial kernel and the end of the call): 64 / (D/8)
    // pairs per wave, 4 waves per workgroup, one round trip.  Few pairs keep one
    // wave per pair, which spreads a small merge over more waves.
    const int nsl = mp.num_splits <= 2 ? 2 : mp.num_splits <= 4 ? 4 : 8;
    switch (3 * (nsl == 2 ? 0 : nsl == 4 ? 1 : 2) + (mp.po_kind == 0 ? 0 : mp.po_kind == 1 ? 1 : 2)) {
      case 0: return launch_merge_narrow<QT, D, 0, 2>(mp, pairs, stream);
      case 1: return launch_merge_narrow<QT, D, 1, 2>(mp, pairs, stream);
      case 2: return launch_merge_narrow<QT, D, 2, 2>(mp, pairs, stream);
      case 3: return launch_merge_narrow<QT, D, 0, 4>(mp, pairs, stream);
      case 4: return launch_merge_narrow<QT, D, 1, 4>(mp, pairs, stream);
      case 5: return launch_merge_narrow<QT, D, 2, 4>(mp, pairs, stream);
      case 6: return launch_merge_narrow<QT, D, 0, 8>(mp, pairs, stream);
      case 7: return launch_merge_narrow<QT, D, 1, 8>(mp, pairs, stream);
      default: return launch_merge_narrow<QT, D, 2, 8>(mp, pairs, stream);
    }
  }
  switch (merge_waves_per_pair(mp.num_splits, D)) {
    case 1: return launch_merge_wpp<QT, D, 1>(mp, pairs, stream);
    case 2: return launch_merge_wpp<QT, D, 2>(mp, pairs, stream);
    case 4: return launch_merge_wpp<QT, D, 4>(mp, pairs, stream);
    case 8: return launch_merge_wpp<QT, D, 8>(mp, pairs, stream);
    default: return launch_merge_wpp<QT, D, 16>(mp, pairs, stream);
  }
}

// Tokens of a sequence the kernels may touch: the workspace's splits and,
// with a block table, its row length (a CSR page list is bounded per
// sequence inside the kernel).
int length_cap(const l20_pd_fp8_args &a, int num_splits) {
  const int64_t by_splits = (int64_t)num_splits * a.split_size;
  if (a.page_indptr) return (int)by_splits;
  return (int)std::min<int64_t>(by_splits, (int64_t)a.bt_max_pages * a.page_size);
}

l20pd::PartialParams partial_params(const l20_pd_fp8_args &a, int n_s) {
  l20pd::PartialParams pp;
  memset(&pp, 0, sizeof(pp));
  pp.q = a.query;
  pp.q_srow = a.q_stride_row;
  pp.q_shead = a.q_stride_head;
  // The kernels address the caches in bytes.
  const int64_t es = (a.kv_dtype == L20_PD_KV_FP16 || a.kv_dtype == L20_PD_KV_BF16) ? 2 : 1;
  // Pages of 16 m tokens are read as m 16-token sub-pages (contiguous, as
  // check_args requires): m times the pages, each 16 token strides apart.
  const int m = a.page_size / 16;
  pp.page_mult = m;
  pp.page_magic = m > 1 ? (unsigned int)((((uint64_t)1 << 32) + m - 1) / m) : 0u;
  pp.k = a.key_cache;
  pp.k_spage = (m == 1 ? a.k_stride_page : 16 * a.k_stride_token) * es;
  pp.k_stok32 = (int)(a.k_stride_token * es);
  pp.k_shead32 = (int)(a.k_stride_head * es);
  pp.v = a.value_cache;
  pp.v_spage = (m == 1 ? a.v_stride_page : 16 * a.v_stride_token) * es;
  pp.v_stok32 = (int)(a.v_stride_token * es);
  pp.v_shead32 = (int)(a.v_stride_head * es);
  // Bytes one KV-head slice of a page can touch: the buffer range of its loads.
  pp.k_extent = (int)((15 * a.k_stride_token + (int64_t)(a.num_kv_heads - 1) * a.k_stride_head + a.head_dim) * es);
  pp.v_extent = (int)((15 * a.v_stride_token + (int64_t)(a.num_kv_heads - 1) * a.v_stride_head + a.head_dim) * es);
  pp.bt = a.block_table;
  pp.bt_srow = a.bt_stride_row;
  pp.seq_lens = a.seq_lens;
  pp.num_pages = a.num_pages * m;
  pp.po = a.partial_output;
  pp.po_srow = a.po_stride_row;
  pp.po_shead = a.po_stride_head;
  pp.po_ssplit = a.po_stride_split;
  pp.pm = a.partial_max;
  pp.pm_srow = a.pm_stride_row;
  pp.pm_shead = a.pm_stride_head;
  pp.pm_ssplit = a.pm_stride_split;
  pp.pl = a.partial_sum;
  pp.pl_srow = a.ps_stride_row;
  pp.pl_shead = a.ps_stride_head;
  pp.pl_ssplit = a.ps_stride_split;
  pp.out = a.output;
  pp.o_srow = a.o_stride_row;
  pp.o_shead = a.o_stride_head;
  pp.lse = a.lse;
  pp.lse_srow = a.lse_stride_row;
  pp.lse_shead = a.lse_stride_head;
  pp.k_scale = a.k_scale;
  pp.v_scale = a.v_scale;
  pp.k_scale_ph = a.k_scale_per_head;
  pp.v_scale_ph = a.v_scale_per_head;
  const float sm = a.softmax_scale > 0.0f ? a.softmax_scale : 1.0f / sqrtf((float)a.head_dim);
  pp.qk_scale_log2 = sm * l20pd::kLog2e;
  pp.q_len = a.q_len;
  pp.num_q_heads = a.num_q_heads;
  pp.num_kv_heads = a.num_kv_heads;
  pp.group = a.num_q_heads / a.num_kv_heads;
  pp.split_size = a.split_size;
  pp.num_splits = n_s > 0 ? n_s : 1;
  pp.po_kind = a.partial_dtype == L20_PD_FP32 ? 0 : a.partial_dtype == L20_PD_FP16 ? 1 : 2;
  pp.l_cap = length_cap(a, pp.num_splits);
  pp.batch = a.batch;
  pp.bt_pages = a.bt_max_pages;
  pp.indptr = a.page_indptr;
  pp.tree = a.tree_mask;
  pp.tree_sb = a.tree_mask_stride_batch;

  return pp;
}

// Work-queue counter slots of the split schedule, per device.  Launches on one
// stream run in order and share the stream's slot; a launch captured into a
// graph takes the next slot of a separate pool, since the graph may replay on
// any stream.  More streams in use at once than eager slots share slots
// (least recently used first; the kernel reports launches whose claims then
// interleave).  A fixed table: taking a slot allocates nothing.  Devices past
// kSlotDevices share the table of device % kSlotDevices (their counters are
// still their own; only the choice of slot is shared).
constexpr int kCaptureSlots = 16;
constexpr int kEagerSlots = l20pd::kQueueSlots - kCaptureSlots;
constexpr int kSlotDevices = 64;
struct SlotEntry {
  void *stream;   // the stream holding this slot, or null
  uint64_t used;  // last use (g_slot_clock), 0 for a free slot
};
std::mutex g_slot_mu;
SlotEntry g_slots[kSlotDevices][kEagerSlots];
uint64_t g_slot_clock = 0;
std::atomic<unsigned int> g_capture_seq{0};
// Launch numbers, mixed into each launch's work-queue tag.
std::atomic<unsigned int> g_launch_seq{0};

int counter_slot(hipStream_t stream) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusActive)
    return kEagerSlots + (int)(g_capture_seq.fetch_add(1u) % kCaptureSlots);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  SlotEntry *tab = g_slots[dev % kSlotDevices];
  std::lock_guard<std::mutex> lock(g_slot_mu);
  const uint64_t now = ++g_slot_clock;
  int lru = 0;
  for (int sl = 0; sl < kEagerSlots; ++sl) {
    if (tab[sl].used != 0 && tab[sl].stream == (void *)stream) {
      tab[sl].used = now;
      return sl;
    }
    if (tab[sl].used < tab[lru].used) lru = sl;  // a free slot (used 0) wins
  }
  tab[lru].stream = (void *)stream;
  tab[lru].used = now;
  return lru;
}

// Poll limit of the partial kernel's hand-off waits, per device (set by
// l20_pd_set_spin_limit, passed to every launch as a kernel argument).
constexpr int kSpinDevices = 64;
std::atomic<unsigned int> g_spin_limit[kSpinDevices];
unsigned int spin_limit() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kSpinDevices) return l20pd::kSpinLimit;
  const unsigned int v = g_spin_limit[dev].load(std::memory_order_relaxed);
  return v ? v : l20pd::kSpinLimit;
}

l20pd::MergeParams merge_params(const l20_pd_fp8_args &a, int num_splits) {
  l20pd::MergeParams mp;
  memset(&mp, 0, sizeof(mp));
  mp.po = a.partial_output;
  mp.po_srow = a.po_stride_row;
  mp.po_shead = a.po_stride_head;
  mp.po_ssplit = a.po_stride_split;
  mp.pm = a.partial_max;
  mp.pm_srow = a.pm_stride_row;
  mp.pm_shead = a.pm_stride_head;
  mp.pm_ssplit = a.pm_stride_split;
  mp.pl = a.partial_sum;
  mp.pl_srow = a.ps_stride_row;
  mp.pl_shead = a.ps_stride_head;
  mp.pl_ssplit = a.ps_stride_split;
  mp.seq_lens = a.seq_lens;
  mp.out = a.output;
  mp.o_srow = a.o_stride_row;
  mp.o_shead = a.o_stride_head;
  mp.lse = a.lse;
  mp.lse_srow = a.lse_stride_row;
  mp.lse_shead = a.lse_stride_head;
  mp.q_len = a.q_len;
  mp.split_size = a.split_size;
  mp.num_splits = num_splits;
  mp.po_kind = a.partial_dtype == L20_PD_FP32 ? 0 : a.partial_dtype == L20_PD_FP16 ? 1 : 2;
  // Speculative first-group loads when the whole workspace is small (<= 4 MB
  // of o partials) and has slots past the first step: config 2 (2 MB) then
  // merges in one round trip; config 3 (14.7 MB, most rows far below the
  // workspace's split count) and config 1 (every slot in the first step) do not.
  const int64_t po_bytes = (int64_t)a.batch * a.q_len * a.num_q_heads * num_splits * a.head_dim *
                           (mp.po_kind == 0 ? 4 : 2);
  const int first_step = merge_waves_per_pair(num_splits, a.head_dim) * (512 / a.head_dim);
  mp.spec_all = po_bytes <= ((int64_t)4 << 20) && num_splits > first_step ? 1 : 0;
  mp.l_cap = length_cap(a, num_splits);
  mp.rows = a.batch * a.q_len;
  mp.num_q_heads = a.num_q_heads;
  return mp;
}

// Which kernels one call enqueues.
enum Stage { kPartial = 1, kMerge = 2, kBoth = 3 };

// Which cache types an entry point accepts.
enum KvKind { kKvFp8 = 1, kKv16 = 2, kKvAny = 3 };

int32_t run(const l20_pd_fp8_args *a, void *stream_ptr, int stages, int kinds) {
  g_last_error[0] = '\0';
  const int32_t rc = check_args(a);
  if (rc != L20_PD_OK) return rc;
  const bool kv16 = a->kv_dtype == L20_PD_KV_FP16 || a->kv_dtype == L20_PD_KV_BF16;
  const bool e5m2 = a->kv_dtype == L20_PD_KV_FP8_E5M2;
  if (!(kinds & (kv16 ? kKv16 : kKvFp8)))
    return fail(L20_PD_EINVAL, kv16 ? "K/V cache must be torch.float8_e4m3fn"
                                    : "K/V cache must be fp16 or bf16 for this entry point");
  if (a->batch == 0) return L20_PD_OK;
  const int n_s = l20_pd_num_splits(a->max_seq_len, a->split_size);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const int group = a->num_q_heads / a->num_kv_heads;
  const int nqt = (group * a->q_len + 15) / 16;
  l20pd::PartialParams pp = partial_params(*a, n_s);
  pp.queue_slot = counter_slot(stream);
  pp.spin_cap = spin_limit();
  pp.launch_tag = g_launch_seq.fetch_add(1u, std::memory_order_relaxed);
  const l20pd::MergeParams mp = merge_params(*a, pp.num_splits);
  const bool bf16 = a->query_dtype == L20_PD_BF16;
  const int rows = a->batch * a->q_len;
  hipError_t e = hipSuccess;
  if (stages == kBoth && fused_fits(*a, pp, nqt, kv16)) {
    const int D = a->head_dim, B = a->batch, H = a->num_kv_heads;
    if (kv16)
      e = bf16 ? launch_fused<__bf16, 1>(pp, D, nqt, B, H, stream) : launch_fused<_Float16, 1>(pp, D, nqt, B, H, stream);
    else if (e5m2)
      e = bf16 ? launch_fused<__bf16, 2>(pp, D, nqt, B, H, stream) : launch_fused<_Float16, 2>(pp, D, nqt, B, H, stream);
    else
      e = bf16 ? launch_fused<__bf16, 0>(pp, D, nqt, B, H, stream) : launch_fused<_Float16, 0>(pp, D, nqt, B, H, stream);
    if (e != hipSuccess) {
      snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s", hipGetErrorString(e));
      return L20_PD_ELAUNCH;
    }
    return L20_PD_OK;
  }
  if ((stages & kPartial) && fused_split_fits(*a, pp, nqt, kv16)) {
    const int D = a->head_dim, B = a->batch, H = a->num_kv_heads;
    l20pd::PartialParams ps = pp;
    ps.fused_split = a->split_size;
    if (kv16)
      e = bf16 ? launch_fused<__bf16, 1>(ps, D, nqt, B, H, stream) : launch_fused<_Float16, 1>(ps, D, nqt, B, H, stream);
    else if (e5m2)
      e = bf16 ? launch_fused<__bf16, 2>(ps, D, nqt, B, H, stream) : launch_fused<_Float16, 2>(ps, D, nqt, B, H, stream);
    else
      e = bf16 ? launch_fused<__bf16, 0>(ps, D, nqt, B, H, stream) : launch_fused<_Float16, 0>(ps, D, nqt, B, H, stream);
  } else if (stages & kPartial) {
    const int D = a->head_dim, B = a->batch, H = a->num_kv_heads;
    if (kv16)
      e = bf16 ? launch_partial_shape<__bf16, 1>(pp, D, nqt, B, H, stream)
               : launch_partial_shape<_Float16, 1>(pp, D, nqt, B, H, stream);
    else if (e5m2)
      e = bf16 ? launch_partial_shape<__bf16, 2>(pp, D, nqt, B, H, stream)
               : launch_partial_shape<_Float16, 2>(pp, D, nqt, B, H, stream);
    else
      e = bf16 ? launch_partial_shape<__bf16, 0>(pp, D, nqt, B, H, stream)
               : launch_partial_shape<_Float16, 0>(pp, D, nqt, B, H, stream);
  }
  // With a single split every row is finished by the partial kernel.
  if (e == hipSuccess && (stages & kMerge) && n_s > 1) {
    if (a->head_dim == 128)
      e = bf16 ? launch_merge<__bf16, 128>(mp, rows, a->num_q_heads, stream)
               : launch_merge<_Float16, 128>(mp, rows, a->num_q_heads, stream);
    else
      e = bf16 ? launch_merge<__bf16, 64>(mp, rows, a->num_q_heads, stream)
               : launch_merge<_Float16, 64>(mp, rows, a->num_q_heads, stream);
  }
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s", hipGetErrorString(e));
    return L20_PD_ELAUNCH;
  }
  return L20_PD_OK;
}

// ---------------------------------------------------------------------------
// Library-held scratch for the allocation-free entry point
// ---------------------------------------------------------------------------
// The split partials (o / l, m, l) of l20_pd_fp8_e4m3_split_out_noalloc live
// in this array instead of a caller workspace.  Each device the library runs
// on holds its own copy for the life of the process.  Host code never passes
// the array's name to a kernel or a copy (on the host it is only a stand-in
// for the symbol): the device address comes from hipGetSymbolAddress, looked
// up once per device with that device current, and kept in g_scratch_ptr.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array (nullptr after a
// failed lookup, with the error recorded).
void *scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(L20_PD_ELAUNCH, "noalloc: no current HIP device (or device index >= 64)");
    return nullptr;
  }
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (p) return p;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    snprintf(g_last_error, sizeof(g_last_error), "noalloc: hipGetSymbolAddress(scratch) failed: %s",
             hipGetErrorString(e));
    return nullptr;
  }
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

// Error reporting for the other translation units of the library.
namespace l20pd_host {
int32_t set_error(int32_t code, const char *msg) { return fail(code, msg); }
void clear_error() { g_last_error[0] = '\0'; }
}  // namespace l20pd_host

extern "C" {

int32_t l20_pd_abi_version(void) { return L20_PD_ABI_VERSION; }

const char *l20_pd_last_error(void) { return g_last_error; }

int32_t l20_pd_num_splits(int32_t max_seq_len, int32_t split_size) {
  if (max_seq_len <= 0 || split_size <= 0) return 0;
  return (max_seq_len + split_size - 1) / split_size;
}

int32_t l20_pd_fp8_e4m3_check(const l20_pd_fp8_args *args) {
  g_last_error[0] = '\0';
  return check_args(args);
}

int32_t l20_pd_default_split_size(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len, int32_t cu_count) {
  // Measured on MI355X over the benchmark workloads: 512-token splits (the
  // reference hook's default) for ragged serving batches, 1024 for long
  // contexts (fewer partials to merge), and at least ~8 splits per sequence
  // for short contexts, where the launch is latency-bound.
  if (max_seq_len > 32768) return 1024;
  // Beyond the single launch's reach (1024 tokens), a batch whose 256-, 512-
  // or 1024-token (split, sequence, KV head) triples (the first that does)
  // fill the CUs once by the split mode's rule runs the single-launch
  // kernel's split mode at that split.
  if (max_seq_len > 1024) {
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    for (const int32_t sp : {256, 512, 1024}) {
      const int64_t triples = (int64_t)batch * (num_kv_heads > 0 ? num_kv_heads : 1) * l20_pd_num_splits(max_seq_len, sp);
      if (split_mode_fills(sp, triples, cus)) return sp;
    }
  }
  int32_t s = 512;
  while (s > 64 && (int64_t)s * 8 > max_seq_len) s >>= 1;
  // Double the split while that lets every (sequence, split) item of a batch
  // at max_seq_len start in the first round of the persistent grid (one item
  // per workgroup: no item transition, which costs a query reload in the
  // two-tile kernel).  Grid estimate: CUs x 8 waves (2 per SIMD at the
  // kernel's occupancy) / waves per workgroup.  Verify shape (64 x 4096,
  // 8 KV heads): 512 -> 1024, 142 -> 126 us per partial launch.
  const int64_t grid = (int64_t)(cu_count > 0 ? cu_count : 256) *
                       std::max(1, 8 / partial_waves(num_kv_heads > 0 ? num_kv_heads : 1));
  while (s < 1024 && (int64_t)batch * l20_pd_num_splits(max_seq_len, s) > grid &&
         (int64_t)batch * l20_pd_num_splits(max_seq_len, 2 * s) <= grid)
    s <<= 1;
  // Halve the split while the items still fill at most half the grid: a
  // short-context batch that leaves most workgroup slots empty streams with
  // too few bytes in flight (32 x 2048 tokens, 2 KV heads: 256 -> 128, 18.6 ->
  // 17.1 us per call; 64 fills the whole grid and is slower again, 19.2 us).
  while (s > 64 && (int64_t)batch * l20_pd_num_splits(max_seq_len, s / 2) <= grid / 2) s >>= 1;
  return s;
}

int32_t l20_pd_fp8_e4m3_split_out(const l20_pd_fp8_args *a, void *stream) { return run(a, stream, kBoth, kKvFp8); }

int32_t l20_pd_set_spin_limit(uint32_t polls) {
  g_last_error[0] = '\0';
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kSpinDevices) {
    snprintf(g_last_error, sizeof(g_last_error), "l20_pd_set_spin_limit: %s",
             e != hipSuccess ? hipGetErrorString(e) : "device index >= 64");
    return L20_PD_ELAUNCH;
  }
  g_spin_limit[dev].store(polls ? polls : l20pd::kSpinLimit, std::memory_order_relaxed);
  return L20_PD_OK;
}

int32_t l20_pd_single_launch(const l20_pd_fp8_args *a) {
  g_last_error[0] = '\0';
  const int32_t rc = check_args(a);
  if (rc != L20_PD_OK) return -rc;
  if (a->batch == 0) return 0;
  const bool kv16 = a->kv_dtype == L20_PD_KV_FP16 || a->kv_dtype == L20_PD_KV_BF16;
  const int n_s = l20_pd_num_splits(a->max_seq_len, a->split_size);
  const int nqt = (a->num_q_heads / a->num_kv_heads * a->q_len + 15) / 16;
  const l20pd::PartialParams pp = partial_params(*a, n_s);
  return fused_fits(*a, pp, nqt, kv16) ? 1 : fused_split_fits(*a, pp, nqt, kv16) ? 2 : 0;
}

int32_t l20_pd_set_queue_counters(uint64_t value) {
  g_last_error[0] = '\0';
  unsigned long long words[l20pd::kQueueSlots][8] = {};
  static_assert(sizeof(words) == sizeof(l20pd::g_pd_queue), "one word per counter line");
  for (int sl = 0; sl < l20pd::kQueueSlots; ++sl) words[sl][0] = value;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = hipMemcpyToSymbol(HIP_SYMBOL(l20pd::g_pd_queue), words, sizeof(words), 0, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "l20_pd_set_queue_counters: %s", hipGetErrorString(e));
    return L20_PD_ELAUNCH;
  }
  return L20_PD_OK;
}

int32_t l20_pd_device_errors(int32_t clear) {
  g_last_error[0] = '\0';
  unsigned int err[l20pd::kQueueSlots];
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpyFromSymbol(err, HIP_SYMBOL(l20pd::g_pd_error), sizeof(err), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "l20_pd_device_errors: %s", hipGetErrorString(e));
    return -L20_PD_ELAUNCH;
  }
  unsigned int all = 0;
  for (int sl = 0; sl < l20pd::kQueueSlots; ++sl) all |= err[sl];
  if (clear) {
    // A launch that gave up (or two that shared a slot) may have left a
    // work-queue counter mid-way: every slot's counter and error word start
    // from zero again.
    static const unsigned int zero[sizeof(l20pd::g_pd_queue) / sizeof(unsigned int)] = {0};
    e = hipMemcpyToSymbol(HIP_SYMBOL(l20pd::g_pd_queue), zero, sizeof(l20pd::g_pd_queue), 0, hipMemcpyHostToDevice);
    if (e == hipSuccess)
      e = hipMemcpyToSymbol(HIP_SYMBOL(l20pd::g_pd_error), zero, sizeof(l20pd::g_pd_error), 0, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      snprintf(g_last_error, sizeof(g_last_error), "l20_pd_device_errors: %s", hipGetErrorString(e));
      return -L20_PD_ELAUNCH;
    }
  }
  return (int32_t)all;
}

int32_t l20_pd_fp8_e4m3_split_out_noalloc(const l20_pd_fp8_args *a, void *stream) {
  g_last_error[0] = '\0';
  if (!a) return fail(L20_PD_EINVAL, "null argument block");
  l20_pd_fp8_args c = *a;
  c.partial_output = nullptr;
  c.partial_max = nullptr;
  c.partial_sum = nullptr;
  c.partial_splits = 0;
  const int32_t n_s = l20_pd_num_splits(c.max_seq_len, c.split_size);
  // Shapes the checks reject anyway need no scratch; run() reports them.
  const bool sane = c.batch > 0 && c.q_len >= 1 && c.num_q_heads > 0 && (c.head_dim == 64 || c.head_dim == 128);
  if (n_s > 1 && sane) {
    // fp32 partials [rows, Hq, n_s, D] then m and l [rows, Hq, n_s], each 256-byte aligned
    const double pairs = (double)c.batch * c.q_len * c.num_q_heads * n_s;
    if (pairs * (c.head_dim + 2) * 4.0 + 768.0 > (double)kScratchBytes) {
      char msg[256];
      snprintf(msg, sizeof(msg),
               "noalloc: the split partials need %.0f bytes, more than the %zu-byte scratch; use "
               "l20_pd_fp8_e4m3_split_out with a workspace",
               pairs * (c.head_dim + 2) * 4.0, kScratchBytes);
      return fail(L20_PD_EINVAL, msg);
    }
    unsigned char *base = static_cast<unsigned char *>(scratch_ptr());
    if (!base) return L20_PD_ELAUNCH;
    const size_t np = (size_t)pairs;
    const size_t o_bytes = align256(np * (size_t)c.head_dim * 4);
    const size_t ml_bytes = align256(np * 4);
    c.partial_output = base;
    c.partial_dtype = L20_PD_FP32;
    c.po_stride_split = c.head_dim;
    c.po_stride_head = (int64_t)n_s * c.head_dim;
    c.po_stride_row = (int64_t)c.num_q_heads * n_s * c.head_dim;
    c.partial_splits = n_s;
    c.partial_max = reinterpret_cast<float *>(base + o_bytes);
    c.partial_sum = reinterpret_cast<float *>(base + o_bytes + ml_bytes);
    c.pm_stride_split = c.ps_stride_split = 1;
    c.pm_stride_head = c.ps_stride_head = n_s;
    c.pm_stride_row = c.ps_stride_row = (int64_t)c.num_q_heads * n_s;
  }
  return run(&c, stream, kBoth, kKvFp8);
}

int32_t l20_pd_split_out(const l20_pd_fp8_args *a, void *stream) { return run(a, stream, kBoth, kKv16); }

int32_t l20_pd_fp8_e4m3_partial(const l20_pd_fp8_args *a, void *stream) { return run(a, stream, kPartial, kKvAny); }

int32_t l20_pd_fp8_e4m3_merge(const l20_pd_fp8_args *a, void *stream) { return run(a, stream, kMerge, kKvAny); }

int32_t l20_pd_fp8_e4m3_dequant_f32(const uint8_t *src, float *dst, int64_t n, float scale, void *stream) {
  g_last_error[0] = '\0';
  if (n < 0 || (n > 0 && (!src || !dst))) return fail(L20_PD_EINVAL, "invalid dequant arguments");
  if (n == 0) return L20_PD_OK;
  const int64_t threads = (n + 3) / 4;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return fail(L20_PD_EINVAL, "dequant size too large");
  hipLaunchKernelGGL(l20pd::dequant_f32_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), src, dst, n, scale);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s", hipGetErrorString(e));
    return L20_PD_ELAUNCH;
  }
  return L20_PD_OK;
}

int32_t l20_pd_fp8_e4m3_dequant_bf16(const uint8_t *src, uint16_t *dst, int64_t n, void *stream) {
  g_last_error[0] = '\0';
  if (n < 0 || (n > 0 && (!src || !dst))) return fail(L20_PD_EINVAL, "invalid dequant arguments");
  if (n == 0) return L20_PD_OK;
  const int64_t threads = (n + 3) / 4;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return fail(L20_PD_EINVAL, "dequant size too large");
  hipLaunchKernelGGL(l20pd::dequant_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), src, dst, n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s", hipGetErrorString(e));
    return L20_PD_ELAUNCH;
  }
  return L20_PD_OK;
}

int32_t l20_pd_stream_read(const void *src, int64_t bytes, int32_t *sink, int32_t blocks, void *stream) {
  g_last_error[0] = '\0';
  if (!src || !sink || bytes < 0 || bytes % 16 || ((uintptr_t)src % 16) || blocks <= 0)
    return fail(L20_PD_EINVAL, "stream_read needs a 16-byte aligned buffer, a multiple of 16 bytes and blocks > 0");
  // chunks of whole 4 KiB units, each below 2 GiB (the buffer range)
  const int64_t chunk = ((bytes + blocks - 1) / blocks + 4095) / 4096 * 4096;
  if (chunk >= ((int64_t)1 << 31)) return fail(L20_PD_EINVAL, "stream_read: more blocks needed (chunk >= 2 GiB)");
  hipLaunchKernelGGL(l20pd::stream_read_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint8_t *>(src), bytes, chunk, sink);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s", hipGetErrorString(e));
    return L20_PD_ELAUNCH;
  }
  return L20_PD_OK;
}

int32_t l20_pd_stream_copy(const void *src, void *dst, int64_t bytes, int32_t blocks, void *stream) {
  g_last_error[0] = '\0';
  if (!src || !dst || bytes < 0 || bytes % 16 || ((uintptr_t)src % 16) || ((uintptr_t)dst % 16) || blocks <= 0)
    return fail(L20_PD_EINVAL, "stream_copy needs 16-byte aligned buffers, a multiple of 16 bytes and blocks > 0");
  hipLaunchKernelGGL(l20pd::stream_copy_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const l20pd::i32x4 *>(src), reinterpret_cast<l20pd::i32x4 *>(dst), bytes / 16);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s", hipGetErrorString(e));
    return L20_PD_ELAUNCH;
  }
  return L20_PD_OK;
}

}  // extern "C"
