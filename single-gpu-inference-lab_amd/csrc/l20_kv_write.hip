// Paged KV-cache producer for MI355X (gfx950): rotary embedding of Q and K
// and the paged write of K and V into fp8 (OCP e4m3fn) or 16-bit caches.
//
//  kv_rope_write8<T, CT, CS>   the fast path: every Q and K head row of the
//    call is one row of the work; a lane owns eight contiguous dims (16-byte
//    loads and stores), D/8 lanes a row, and each lane takes two rows with
//    all their loads issued before any arithmetic.  A neox pair partner lies
//    half/8 lanes away in the same row and is exchanged with a lane shuffle;
//    cos and sin arrive as 8 (neox) or 4 (interleaved) consecutive values.
//    Taken when rows, caches and the cos/sin table are 16-byte aligned,
//    head_dim % 8 == 0 and, for neox, rotary_dim % 16 == 0.  Row loads and
//    all row and cache stores are non-temporal: every byte is touched once
//    per call and each wave writes whole 128-byte lines (70.3 vs 75.2 us for
//    a 16K-token chunk of the config-3 shape).
//
//  kv_rope_write<T, CT>   the general path: grid (num_tokens, ceil(max(Hq, Hkv) / 4)), 4 waves.
//    Wave w of workgroup (t, g) owns head h = 4 g + w of token t; lane l owns
//    the four contiguous dims [4 l, 4 l + 4) (head_dim <= 256).  A neox pair
//    partner lies rotary_dim / 2 dims away (another lane's four dims, loaded
//    directly: every load of the wave precedes its stores, so the in-place
//    update is safe); an interleaved partner lies inside the lane's four dims.
//    Arithmetic in fp32 with contraction off -- each product and the sum are
//    rounded separately -- then rounded to the model dtype.  fp8 caches take
//    RNE_e4m3fn(clamp(x / scale, +-448)) via v_cvt_pk_fp8_f32 (one dword per
//    lane); 16-bit caches take the dtype value (8 bytes per lane).
//
//  kv_amax<T> + kv_scales_finalize   one workgroup per (KV head, K or V)
//    scans every token (no atomics, deterministic), then one workgroup turns
//    the maxima into scales.
//
// Reference semantics (paths relative to the reference repo root):
//   integrations/vllm/l20_rope_kv.py:26-137 (interleaved), :140-253 (neox),
//   :256-309 (entry point; 16-bit caches only there);
//   scripts/smoke_cuda_paged_fp8_decode_op.py:13-19 (the fp8 quantiser).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <type_traits>

#include "l20_kv_write.h"

// Error reporting shared with the decode entry points (l20_pd_last_error).
namespace l20pd_host {
int32_t set_error(int32_t code, const char *msg);
void clear_error();
}  // namespace l20pd_host

namespace l20kv {

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kFp8Max = 448.0f;

struct Params {
  void *q;
  int64_t q_st, q_sh;
  int hq;
  void *k;
  int64_t k_st, k_sh;
  const void *v;
  int64_t v_st, v_sh;
  const int64_t *pos;
  const void *cs;
  int64_t cs_sp;
  int cs_dtype;  // 0 bf16, 1 fp16, 2 fp32
  int rot, neox;
  const int64_t *slots;
  void *kc;
  int64_t kc_sp, kc_st, kc_sh;
  void *vc;
  int64_t vc_sp, vc_st, vc_sh;
  int64_t num_pages;
  float k_scale, v_scale;
  const float *k_scale_ph, *v_scale_ph;
  int tokens, hkv, d;
};

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

// Four consecutive elements of type T (8 bytes) as fp32.
template <typename T> __device__ __forceinline__ void load4(const T *p, float (&x)[4]) {
  const i32x2 w = *reinterpret_cast<const i32x2 *>(p);
  const T *e = reinterpret_cast<const T *>(&w);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = to_f32(e[i]);
}

// Four fp32 -> four T (RNE), packed as two dwords.
template <typename T> __device__ __forceinline__ i32x2 pack4(const float (&x)[4]);
template <> __device__ __forceinline__ i32x2 pack4<__bf16>(const float (&x)[4]) {
  return i32x2{__builtin_bit_cast(int, __builtin_convertvector(f32x2{x[0], x[1]}, bf16x2)),
               __builtin_bit_cast(int, __builtin_convertvector(f32x2{x[2], x[3]}, bf16x2))};
}
template <> __device__ __forceinline__ i32x2 pack4<_Float16>(const float (&x)[4]) {
  return i32x2{__builtin_bit_cast(int, __builtin_convertvector(f32x2{x[0], x[1]}, f16x2)),
               __builtin_bit_cast(int, __builtin_convertvector(f32x2{x[2], x[3]}, f16x2))};
}

// The fp32 values of four packed T (what a store then load would give).
template <typename T> __device__ __forceinline__ void unpack4(i32x2 w, float (&x)[4]) {
  const T *e = reinterpret_cast<const T *>(&w);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = to_f32(e[i]);
}

__device__ __forceinline__ float cs_load(const Params &p, int64_t position, int idx) {
  const int64_t off = position * p.cs_sp + idx;
  if (p.cs_dtype == 2) return reinterpret_cast<const float *>(p.cs)[off];
  if (p.cs_dtype == 1) return (float)reinterpret_cast<const _Float16 *>(p.cs)[off];
  return (float)reinterpret_cast<const __bf16 *>(p.cs)[off];
}

// Rotate the lane's four dims [e0, e0 + 4) of one head row in fp32.
template <typename T>
__device__ __forceinline__ void rope4(const Params &p, const T *row, int64_t position, int e0, float (&x)[4]) {
#pragma clang fp contract(off)
  load4(row + e0, x);
  if (e0 >= p.rot) return;
  const int half = p.rot >> 1;
  float pr[4], c[4], s[4], sg[4];
  if (p.neox) {
    const bool first = e0 < half;
    load4(row + (first ? e0 + half : e0 - half), pr);
    const int t0 = first ? e0 : e0 - half;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = cs_load(p, position, t0 + i);
      s[i] = cs_load(p, position, half + t0 + i);
      sg[i] = first ? -1.0f : 1.0f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = x[i ^ 1];
      c[i] = cs_load(p, position, (e0 + i) >> 1);
      s[i] = cs_load(p, position, half + ((e0 + i) >> 1));
      sg[i] = (i & 1) ? 1.0f : -1.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = x[i] * c[i];
    const float b = (pr[i] * s[i]) * sg[i];
    x[i] = a + b;
  }
}

// ---- fast path helpers: eight consecutive elements of T as one 16-byte word ----
template <typename T> __device__ __forceinline__ void unpack8(i32x4 w, float (&x)[8]) {
  const T *e = reinterpret_cast<const T *>(&w);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = to_f32(e[i]);
}
template <typename T> __device__ __forceinline__ i32x4 pack8(const float (&x)[8]) {
  const float lo[4] = {x[0], x[1], x[2], x[3]};
  const float hi[4] = {x[4], x[5], x[6], x[7]};
  const i32x2 a = pack4<T>(lo), b = pack4<T>(hi);
  return i32x4{a[0], a[1], b[0], b[1]};
}
// n (4 or 8) consecutive cos/sin values from a table of CS type (0 bf16, 1 fp16, 2 fp32).
template <int CS, int N> __device__ __forceinline__ void load_cs(const void *base, int64_t off, float (&c)[8]) {
  if constexpr (CS == 2) {
    const float *src = reinterpret_cast<const float *>(base) + off;
    const f32x4 a = *reinterpret_cast<const f32x4 *>(src);
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = a[i];
    if constexpr (N == 8) {
      const f32x4 b = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) c[4 + i] = b[i];
    }
  } else {
    typedef typename std::conditional<CS == 0, __bf16, _Float16>::type E;
    const E *src = reinterpret_cast<const E *>(base) + off;
    if constexpr (N == 8) {
      unpack8<E>(*reinterpret_cast<const i32x4 *>(src), c);
    } else {
      float q[4];
      load4(src, q);
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = q[i];
    }
  }
}

// Four values -> four e4m3fn codes in one dword: RNE of clamp(x / scale).
__device__ __forceinline__ int quant4(const float (&x)[4], float scale) {
  float y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i] = fminf(fmaxf(__fdiv_rn(x[i], scale), -kFp8Max), kFp8Max);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w, true);
  return w;
}

constexpr int kRowsPerLane = 2;

// Rows [0, rows_q) are Q head rows (token r / Hq, head r % Hq), the next
// rows_k are K head rows (token r / Hkv): rotated in place, and for K also the
// K and V cache writes.  Four waves; a lane group of lpr = D/8 lanes per row.
template <typename T, int CT, int CS>
__global__ __launch_bounds__(256) void kv_rope_write8(Params p, int64_t rows_q, int64_t rows_all) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lpr = p.d >> 3;     // lanes per row
  const int rpw = 64 / lpr;     // rows per wave and pass
  const int g = lane / lpr;
  const int l = lane - g * lpr;
  const int e0 = 8 * l;
  const int half = p.rot >> 1;
  const bool rot_lane = e0 < p.rot;
  const int64_t first = (int64_t)blockIdx.x * (4 * rpw * kRowsPerLane);

  // ---- loads of all of this lane's rows ----
  i32x4 xw[kRowsPerLane], vw[kRowsPerLane];
  int64_t pos[kRowsPerLane], slot[kRowsPerLane];
  float ksc[kRowsPerLane], vsc[kRowsPerLane];  // the K row's cache scales (loaded with the row)
  T *row[kRowsPerLane];
  int head[kRowsPerLane];
  bool live[kRowsPerLane], is_k[kRowsPerLane];
#pragma unroll
  for (int u = 0; u < kRowsPerLane; ++u) {
    const int64_t r = first + (int64_t)(u * 4 + wave) * rpw + g;
    live[u] = g < rpw && r < rows_all;
    is_k[u] = r >= rows_q;
    int64_t t = 0;
    int h = 0;
    if (live[u]) {
      if (!is_k[u]) {
        t = r / p.hq;
        h = (int)(r - t * p.hq);
        row[u] = reinterpret_cast<T *>(p.q) + t * p.q_st + (int64_t)h * p.q_sh;
      } else {
        const int64_t rk = r - rows_q;
        t = rk / p.hkv;
        h = (int)(rk - t * p.hkv);
        row[u] = reinterpret_cast<T *>(p.k) + t * p.k_st + (int64_t)h * p.k_sh;
        vw[u] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(reinterpret_cast<const T *>(p.v) + t * p.v_st +
                                                 (int64_t)h * p.v_sh + e0));
        slot[u] = p.slots[t];
        if constexpr (CT == 0) {
          ksc[u] = p.k_scale_ph ? p.k_scale_ph[h] : p.k_scale;
          vsc[u] = p.v_scale_ph ? p.v_scale_ph[h] : p.v_scale;
        }
      }
      xw[u] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(row[u] + e0));
      pos[u] = p.pos[t];
    }
    head[u] = h;
  }
  // ---- cos / sin of the lanes' dims ----
  float c[kRowsPerLane][8], sn[kRowsPerLane][8];
#pragma unroll
  for (int u = 0; u < kRowsPerLane; ++u) {
    if (live[u] && rot_lane) {
      const int64_t base = pos[u] * p.cs_sp;
      if (p.neox) {
        const int t0 = e0 < half ? e0 : e0 - half;
        load_cs<CS, 8>(p.cs, base + t0, c[u]);
        load_cs<CS, 8>(p.cs, base + half + t0, sn[u]);
      } else {
        load_cs<CS, 4>(p.cs, base + (e0 >> 1), c[u]);
        load_cs<CS, 4>(p.cs, base + half + (e0 >> 1), sn[u]);
      }
    }
  }
  // ---- rotate, store back, write the caches ----
#pragma unroll
  for (int u = 0; u < kRowsPerLane; ++u) {
    // the neox partner's words, from the lane half/8 away in the same row (every lane shuffles)
    const int src = g * lpr + (e0 < half ? l + (half >> 3) : l - (half >> 3));
    i32x4 pw;
#pragma unroll
    for (int i = 0; i < 4; ++i) pw[i] = __shfl(xw[u][i], (p.neox && rot_lane) ? src : lane);
    if (!live[u]) continue;
    float x[8];
    unpack8<T>(xw[u], x);
    if (rot_lane) {
      float y[8];
      if (p.neox) {
        float pr[8];
        unpack8<T>(pw, pr);
        const float sg = e0 < half ? -1.0f : 1.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float a = x[i] * c[u][i];
          const float b = (pr[i] * sn[u][i]) * sg;
          y[i] = a + b;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float a = x[i] * c[u][i >> 1];
          const float b = (x[i ^ 1] * sn[u][i >> 1]) * ((i & 1) ? 1.0f : -1.0f);
          y[i] = a + b;
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = y[i];
    }
    const i32x4 out = pack8<T>(x);
    __builtin_nontemporal_store(out, reinterpret_cast<i32x4 *>(row[u] + e0));
    if (!is_k[u]) continue;
    const int64_t sl = slot[u];
    const int64_t page = sl >> 4;
    if (sl < 0 || page >= p.num_pages) continue;  // not stored
    const int h = head[u];
    const int64_t ko = page * p.kc_sp + (sl & 15) * p.kc_st + (int64_t)h * p.kc_sh + e0;
    const int64_t vo = page * p.vc_sp + (sl & 15) * p.vc_st + (int64_t)h * p.vc_sh + e0;
    if constexpr (CT == 0) {
      float kv[8], v[8];
      unpack8<T>(out, kv);  // quantise the stored model-dtype values
      unpack8<T>(vw[u], v);
      const float ks = ksc[u], vs = vsc[u];
      const float k_lo[4] = {kv[0], kv[1], kv[2], kv[3]}, k_hi[4] = {kv[4], kv[5], kv[6], kv[7]};
      const float v_lo[4] = {v[0], v[1], v[2], v[3]}, v_hi[4] = {v[4], v[5], v[6], v[7]};
      __builtin_nontemporal_store(i32x2{quant4(k_lo, ks), quant4(k_hi, ks)}, reinterpret_cast<i32x2 *>(reinterpret_cast<uint8_t *>(p.kc) + ko));
      __builtin_nontemporal_store(i32x2{quant4(v_lo, vs), quant4(v_hi, vs)}, reinterpret_cast<i32x2 *>(reinterpret_cast<uint8_t *>(p.vc) + vo));
    } else {
      *reinterpret_cast<i32x4 *>(reinterpret_cast<T *>(p.kc) + ko) = out;
      *reinterpret_cast<i32x4 *>(reinterpret_cast<T *>(p.vc) + vo) = vw[u];
    }
  }
}

template <typename T, int CT>
__global__ __launch_bounds__(256) void kv_rope_write(Params p) {
  const int t = blockIdx.x;
  const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int e0 = 4 * lane;
  if (e0 >= p.d) return;
  const int64_t position = p.pos[t];
  float x[4];
  if (p.q && h < p.hq) {
    T *row = reinterpret_cast<T *>(p.q) + (int64_t)t * p.q_st + (int64_t)h * p.q_sh;
    rope4<T>(p, row, position, e0, x);
    *reinterpret_cast<i32x2 *>(row + e0) = pack4<T>(x);
  }
  if (h >= p.hkv) return;
  T *krow = reinterpret_cast<T *>(p.k) + (int64_t)t * p.k_st + (int64_t)h * p.k_sh;
  rope4<T>(p, krow, position, e0, x);
  const i32x2 kw = pack4<T>(x);
  *reinterpret_cast<i32x2 *>(krow + e0) = kw;
  const int64_t slot = p.slots[t];
  if (slot < 0) return;
  const int64_t page = slot >> 4;
  const int64_t r = slot & 15;
  if (page >= p.num_pages) return;  // outside the cache: nothing to write
  float v[4];
  load4(reinterpret_cast<const T *>(p.v) + (int64_t)t * p.v_st + (int64_t)h * p.v_sh + e0, v);
  const int64_t ko = page * p.kc_sp + r * p.kc_st + (int64_t)h * p.kc_sh + e0;
  const int64_t vo = page * p.vc_sp + r * p.vc_st + (int64_t)h * p.vc_sh + e0;
  if constexpr (CT == 0) {
    float kv[4];
    unpack4<T>(kw, kv);  // quantise the stored model-dtype values
    const float ks = p.k_scale_ph ? p.k_scale_ph[h] : p.k_scale;
    const float vs = p.v_scale_ph ? p.v_scale_ph[h] : p.v_scale;
    *reinterpret_cast<int *>(reinterpret_cast<uint8_t *>(p.kc) + ko) = quant4(kv, ks);
    *reinterpret_cast<int *>(reinterpret_cast<uint8_t *>(p.vc) + vo) = quant4(v, vs);
  } else {
    *reinterpret_cast<i32x2 *>(reinterpret_cast<T *>(p.kc) + ko) = kw;
    *reinterpret_cast<i32x2 *>(reinterpret_cast<T *>(p.vc) + vo) = pack4<T>(v);
  }
}

// amax of the stored K (rotated, dtype-rounded) or of V over all tokens of
// one KV head: workgroup (h, which), 1024 threads, token-strided.
template <typename T>
__global__ __launch_bounds__(1024) void kv_amax(Params p, float *k_out, float *v_out) {
  __shared__ float s_red[16];
  const int h = blockIdx.x;
  const bool is_k = blockIdx.y == 0;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int e0 = 4 * lane;
  float m = 0.0f;
  if (e0 < p.d) {
    for (int t = wave; t < p.tokens; t += 16) {
      const int64_t slot = p.slots[t];
      if (slot < 0 || (slot >> 4) >= p.num_pages) continue;  // not stored
      float x[4];
      if (is_k) {
        const T *row = reinterpret_cast<const T *>(p.k) + (int64_t)t * p.k_st + (int64_t)h * p.k_sh;
        rope4<T>(p, row, p.pos[t], e0, x);
        const i32x2 w = pack4<T>(x);
        unpack4<T>(w, x);
      } else {
        load4(reinterpret_cast<const T *>(p.v) + (int64_t)t * p.v_st + (int64_t)h * p.v_sh + e0, x);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(x[i]));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = 0.0f;
    for (int w = 0; w < 16; ++w) r = fmaxf(r, s_red[w]);
    (is_k ? k_out : v_out)[h] = r;
  }
}

// amax -> max(amax / 448, 1e-12), per head or (per_head = 0) the maximum over heads.
__global__ void kv_scales_finalize(float *k_scales, float *v_scales, int hkv, int per_head) {
  if (threadIdx.x >= 2) return;
  float *s = threadIdx.x == 0 ? k_scales : v_scales;
  float all = 0.0f;
  for (int h = 0; h < hkv; ++h) all = fmaxf(all, s[h]);
  for (int h = 0; h < hkv; ++h) s[h] = fmaxf(__fdiv_rn(per_head ? s[h] : all, kFp8Max), 1e-12f);
}

}  // namespace l20kv

namespace {

using l20pd_host::set_error;

int32_t check(const l20_pd_kv_write_args *a) {
  if (!a) return set_error(L20_PD_EINVAL, "null argument block");
  if (a->dtype != L20_PD_BF16 && a->dtype != L20_PD_FP16)
    return set_error(L20_PD_EINVAL, "query, key and value must be bf16 or fp16");
  if (a->cs_dtype != L20_PD_BF16 && a->cs_dtype != L20_PD_FP16 && a->cs_dtype != L20_PD_FP32)
    return set_error(L20_PD_EINVAL, "cos_sin_cache must be bf16, fp16 or fp32");
  const bool fp8 = a->cache_dtype == L20_PD_KV_FP8_E4M3;
  if (!fp8 && a->cache_dtype != L20_PD_KV_FP16 && a->cache_dtype != L20_PD_KV_BF16)
    return set_error(L20_PD_EINVAL, "unknown K/V cache dtype");
  if (!fp8 && (a->cache_dtype == L20_PD_KV_BF16) != (a->dtype == L20_PD_BF16))
    return set_error(L20_PD_EINVAL, "a 16-bit cache must have the model dtype");
  if (a->head_dim <= 0 || a->head_dim > 256 || a->head_dim % 4)
    return set_error(L20_PD_EINVAL, "head_dim must be a multiple of 4 up to 256");
  if (a->rotary_dim < 0 || a->rotary_dim > a->head_dim || a->rotary_dim % 8)
    return set_error(L20_PD_EINVAL, "invalid cos_sin_cache rotary dimension");
  if (a->num_tokens < 0 || a->num_kv_heads <= 0 || (a->query && a->num_q_heads <= 0))
    return set_error(L20_PD_EINVAL, "token and head counts must be positive");
  if ((int64_t)std::max(a->num_q_heads, a->num_kv_heads) > 65535 * 4)
    return set_error(L20_PD_EINVAL, "too many heads");
  if (a->num_tokens == 0) return L20_PD_OK;
  if (!a->key || !a->value || !a->positions || !a->slot_mapping || !a->key_cache || !a->value_cache ||
      (a->rotary_dim > 0 && !a->cos_sin_cache))
    return set_error(L20_PD_EINVAL, "null tensor pointer");
  // 8-byte row chunks of the 16-bit tensors, 4-byte (fp8) or 8-byte (16-bit) cache chunks
  const uint64_t qkv = (uint64_t)(uintptr_t)a->key | (uint64_t)(uintptr_t)a->value |
                       (uint64_t)(a->k_stride_token * 2) | (uint64_t)(a->k_stride_head * 2) |
                       (uint64_t)(a->v_stride_token * 2) | (uint64_t)(a->v_stride_head * 2) |
                       (a->query ? ((uint64_t)(uintptr_t)a->query | (uint64_t)(a->q_stride_token * 2) |
                                    (uint64_t)(a->q_stride_head * 2))
                                 : 0);
  if (qkv % 8) return set_error(L20_PD_EINVAL, "query/key/value pointers and strides must be 8-byte aligned");
  const int64_t es = fp8 ? 1 : 2;
  const uint64_t cb = (uint64_t)(uintptr_t)a->key_cache | (uint64_t)(uintptr_t)a->value_cache |
                      (uint64_t)(a->kc_stride_page * es) | (uint64_t)(a->kc_stride_token * es) |
                      (uint64_t)(a->kc_stride_head * es) | (uint64_t)(a->vc_stride_page * es) |
                      (uint64_t)(a->vc_stride_token * es) | (uint64_t)(a->vc_stride_head * es);
  if (cb % (uint64_t)(4 * es)) return set_error(L20_PD_EINVAL, "cache pointers and strides must be aligned to 4 elements");
  if (a->num_pages <= 0) return set_error(L20_PD_EINVAL, "K/V cache has no pages");
  return L20_PD_OK;
}

l20kv::Params params(const l20_pd_kv_write_args &a) {
  l20kv::Params p{};
  p.q = a.query;
  p.q_st = a.q_stride_token;
  p.q_sh = a.q_stride_head;
  p.hq = a.query ? a.num_q_heads : 0;
  p.k = a.key;
  p.k_st = a.k_stride_token;
  p.k_sh = a.k_stride_head;
  p.v = a.value;
  p.v_st = a.v_stride_token;
  p.v_sh = a.v_stride_head;
  p.pos = a.positions;
  p.cs = a.cos_sin_cache;
  p.cs_sp = a.cs_stride_position;
  p.cs_dtype = a.cs_dtype == L20_PD_FP32 ? 2 : (a.cs_dtype == L20_PD_FP16 ? 1 : 0);
  p.rot = a.rotary_dim;
  p.neox = a.is_neox != 0;
  p.slots = a.slot_mapping;
  p.kc = a.key_cache;
  p.kc_sp = a.kc_stride_page;
  p.kc_st = a.kc_stride_token;
  p.kc_sh = a.kc_stride_head;
  p.vc = a.value_cache;
  p.vc_sp = a.vc_stride_page;
  p.vc_st = a.vc_stride_token;
  p.vc_sh = a.vc_stride_head;
  p.num_pages = a.num_pages;
  p.k_scale = a.k_scale;
  p.v_scale = a.v_scale;
  p.k_scale_ph = a.k_scale_per_head;
  p.v_scale_ph = a.v_scale_per_head;
  p.tokens = a.num_tokens;
  p.hkv = a.num_kv_heads;
  p.d = a.head_dim;
  return p;
}

// The fast path's layout requirements (16-byte rows and cache chunks, lane-aligned neox halves).
bool fast_path_ok(const l20_pd_kv_write_args &a) {
  if (a.head_dim % 8 || (a.is_neox && a.rotary_dim % 16)) return false;
  const uint64_t qkv = (uint64_t)(uintptr_t)a.key | (uint64_t)(uintptr_t)a.value |
                       (uint64_t)(a.k_stride_token * 2) | (uint64_t)(a.k_stride_head * 2) |
                       (uint64_t)(a.v_stride_token * 2) | (uint64_t)(a.v_stride_head * 2) |
                       (a.query ? ((uint64_t)(uintptr_t)a.query | (uint64_t)(a.q_stride_token * 2) |
                                   (uint64_t)(a.q_stride_head * 2))
                                : 0);
  if (qkv % 16) return false;
  const bool fp8 = a.cache_dtype == L20_PD_KV_FP8_E4M3;
  const int64_t es = fp8 ? 1 : 2;
  const uint64_t cb = (uint64_t)(uintptr_t)a.key_cache | (uint64_t)(uintptr_t)a.value_cache |
                      (uint64_t)(a.kc_stride_page * es) | (uint64_t)(a.kc_stride_token * es) |
                      (uint64_t)(a.kc_stride_head * es) | (uint64_t)(a.vc_stride_page * es) |
                      (uint64_t)(a.vc_stride_token * es) | (uint64_t)(a.vc_stride_head * es);
  if (cb % (uint64_t)(8 * es)) return false;
  if (a.rotary_dim > 0) {
    const int64_t cs_es = a.cs_dtype == L20_PD_FP32 ? 4 : 2;
    const uint64_t cs = (uint64_t)(uintptr_t)a.cos_sin_cache | (uint64_t)(a.cs_stride_position * cs_es) |
                        (uint64_t)(a.rotary_dim / 2 * cs_es);
    // neox: 8 values per 16-byte load; interleaved: 4 values (8 bytes, or 16 for fp32)
    if (cs % (uint64_t)(a.is_neox ? 16 : 4 * cs_es)) return false;
  }
  return true;
}

template <typename T, int CT>
void launch_fast(const l20kv::Params &p, int cs_dtype, int64_t rows_q, int64_t rows_all, hipStream_t s) {
  const int lpr = p.d / 8;
  const int64_t rows_per_wg = (int64_t)4 * (64 / lpr) * l20kv::kRowsPerLane;
  const dim3 grid((unsigned)((rows_all + rows_per_wg - 1) / rows_per_wg));
  if (cs_dtype == 2)
    hipLaunchKernelGGL((l20kv::kv_rope_write8<T, CT, 2>), grid, dim3(256), 0, s, p, rows_q, rows_all);
  else if (cs_dtype == 1)
    hipLaunchKernelGGL((l20kv::kv_rope_write8<T, CT, 1>), grid, dim3(256), 0, s, p, rows_q, rows_all);
  else
    hipLaunchKernelGGL((l20kv::kv_rope_write8<T, CT, 0>), grid, dim3(256), 0, s, p, rows_q, rows_all);
}

int32_t launched() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[256];
    snprintf(msg, sizeof(msg), "HIP launch failed: %s", hipGetErrorString(e));
    return set_error(L20_PD_ELAUNCH, msg);
  }
  return L20_PD_OK;
}

}  // namespace

extern "C" {

int32_t l20_pd_kv_write_check(const l20_pd_kv_write_args *args) {
  l20pd_host::clear_error();
  return check(args);
}

int32_t l20_pd_rope_and_cache(const l20_pd_kv_write_args *a, void *stream) {
  l20pd_host::clear_error();
  const int32_t rc = check(a);
  if (rc != L20_PD_OK || a->num_tokens == 0) return rc;
  const l20kv::Params p = params(*a);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = a->dtype == L20_PD_BF16;
  if (fast_path_ok(*a)) {
    const int64_t rows_q = (int64_t)a->num_tokens * p.hq;
    const int64_t rows_all = rows_q + (int64_t)a->num_tokens * p.hkv;
    const bool fp8 = a->cache_dtype == L20_PD_KV_FP8_E4M3;
    if (bf) {
      if (fp8) launch_fast<__bf16, 0>(p, p.cs_dtype, rows_q, rows_all, s);
      else launch_fast<__bf16, 1>(p, p.cs_dtype, rows_q, rows_all, s);
    } else {
      if (fp8) launch_fast<_Float16, 0>(p, p.cs_dtype, rows_q, rows_all, s);
      else launch_fast<_Float16, 1>(p, p.cs_dtype, rows_q, rows_all, s);
    }
    return launched();
  }
  const int heads = std::max(p.hq, p.hkv);
  const dim3 grid((unsigned)a->num_tokens, (unsigned)((heads + 3) / 4));
  if (a->cache_dtype == L20_PD_KV_FP8_E4M3) {
    if (bf)
      hipLaunchKernelGGL((l20kv::kv_rope_write<__bf16, 0>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((l20kv::kv_rope_write<_Float16, 0>), grid, dim3(256), 0, s, p);
  } else {
    if (bf)
      hipLaunchKernelGGL((l20kv::kv_rope_write<__bf16, 1>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((l20kv::kv_rope_write<_Float16, 1>), grid, dim3(256), 0, s, p);
  }
  return launched();
}

int32_t l20_pd_kv_fp8_scales(const l20_pd_kv_write_args *a, float *k_scales, float *v_scales, int32_t per_head,
                             void *stream) {
  l20pd_host::clear_error();
  const int32_t rc = check(a);
  if (rc != L20_PD_OK) return rc;
  if (!k_scales || !v_scales) return set_error(L20_PD_EINVAL, "null scale output");
  const l20kv::Params p = params(*a);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == L20_PD_BF16)
    hipLaunchKernelGGL((l20kv::kv_amax<__bf16>), dim3((unsigned)a->num_kv_heads, 2), dim3(1024), 0, s, p, k_scales,
                       v_scales);
  else
    hipLaunchKernelGGL((l20kv::kv_amax<_Float16>), dim3((unsigned)a->num_kv_heads, 2), dim3(1024), 0, s, p,
                       k_scales, v_scales);
  int32_t r = launched();
  if (r != L20_PD_OK) return r;
  hipLaunchKernelGGL(l20kv::kv_scales_finalize, dim3(1), dim3(64), 0, s, k_scales, v_scales, a->num_kv_heads,
                     per_head);
  return launched();
}

}  // extern "C"
