"""CPU oracle for the paged KV-cache producer (RoPE + FP8 quantise + paged write).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, and only as
the checker; the product path never calls it.

What it restates (reference file:line, relative to the reference repo root):

* ``rope_and_cache`` -- ``integrations/vllm/l20_rope_kv.py:26-137`` (interleaved
  pairs) and ``:140-253`` (neox halves), entry point ``:256-309``: for every
  token, ``cos = cache[pos, trig]`` and ``sin = cache[pos, half + trig]`` in
  fp32, ``x' = x * cos + (x_pair * sin) * sign`` (sign -1 on the first element
  of a pair) for the first ``rotary_dim`` dims, other dims unchanged; Q and K
  are rotated in place (stored back in their dtype), K and V are written to the
  paged cache at ``slot_mapping[t]`` (page ``slot // 16``, row ``slot % 16``),
  tokens with ``slot < 0`` are skipped.
* FP8 caches (the reference's producer has none: it raises "quantized KV cache
  is not supported", ``l20_rope_kv.py:276-277``): the cached value is the
  rotated K (resp. V) as stored in the model dtype, quantised with the
  reference's rule (``scripts/smoke_cuda_paged_fp8_decode_op.py:13-19``):
  ``RNE_e4m3fn(clamp(x / scale, +-448))`` with a per-tensor or per-KV-head
  scale.  ``fp8_scales`` gives ``max(amax / 448, 1e-12)`` over those values.

How it is pinned (tests/test_kv_write_oracle.py): bf16 rounding against
torch's ``.to(torch.bfloat16)``; the rotation against a float64 complex-number
formulation (``z e^{i theta}``) for both pair layouts, the identity at
``theta = 0`` and composition of two rotations; quantisation through
``paged_fp8_decode_ref.encode_e4m3fn`` (itself pinned against torch); the
scatter by a write-then-gather round trip and by skipped negative slots.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

from oracle import paged_fp8_decode_ref as pd

FP8_MAX = pd.FP8_E4M3FN_MAX


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16 << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to the model dtype ('bf16' or 'fp16'), as float32."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


def rope(x: np.ndarray, cos_sin: np.ndarray, rotary_dim: int, is_neox: bool) -> np.ndarray:
    """Rotate the first ``rotary_dim`` dims of ``x`` [..., D] (float32, unrounded result).

    ``cos_sin`` [..., rotary_dim] holds cos in its first half and sin in its
    second, broadcast over the head axis.  Every product and sum is rounded to
    float32 separately (no fused multiply-add)."""
    x = np.asarray(x, dtype=np.float32)
    out = x.copy()
    half = rotary_dim // 2
    idx = np.arange(rotary_dim)
    if is_neox:
        pair = np.where(idx < half, idx + half, idx - half)
        trig = idx % half
        sign = np.where(idx < half, -1.0, 1.0).astype(np.float32)
    else:
        pair = np.where(idx % 2 == 0, idx + 1, idx - 1)
        trig = idx // 2
        sign = np.where(idx % 2 == 0, -1.0, 1.0).astype(np.float32)
    cos = np.asarray(cos_sin[..., :half], dtype=np.float32)[..., None, :][..., trig]
    sin = np.asarray(cos_sin[..., half:rotary_dim], dtype=np.float32)[..., None, :][..., trig]
    a = (x[..., idx] * cos).astype(np.float32)
    b = ((x[..., pair] * sin).astype(np.float32) * sign).astype(np.float32)
    out[..., :rotary_dim] = (a + b).astype(np.float32)
    return out


def quantize_rows(x: np.ndarray, scale) -> np.ndarray:
    """e4m3fn codes of ``x`` [..., Hkv, D] with a scalar or per-head [Hkv] scale."""
    x = np.asarray(x, dtype=np.float32)
    s = np.asarray(scale, dtype=np.float32).reshape(-1)
    s = s.reshape((-1, 1)) if s.size > 1 else s.reshape(())
    scaled = np.clip((x / s).astype(np.float32), -FP8_MAX, FP8_MAX)
    return pd.encode_e4m3fn(scaled)


def fp8_scales(values: np.ndarray, per_head: bool, floor: float = 1e-12) -> np.ndarray:
    """``max(amax / 448, floor)`` over ``values`` [T, Hkv, D]: one per head or one in total."""
    a = np.abs(np.asarray(values, dtype=np.float32))
    amax = a.max(axis=(0, 2)) if per_head else np.array([a.max()], dtype=np.float32)
    return np.maximum(amax.astype(np.float64) / FP8_MAX, floor).astype(np.float32)


def rope_and_cache(
    query: Optional[np.ndarray],
    key: np.ndarray,
    value: np.ndarray,
    positions: np.ndarray,
    cos_sin_cache: np.ndarray,
    is_neox: bool,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    slot_mapping: np.ndarray,
    *,
    dtype: str,
    cache_fp8: bool,
    k_scale=1.0,
    v_scale=1.0,
) -> Tuple[Optional[np.ndarray], np.ndarray, np.ndarray, np.ndarray]:
    """Returns ``(query', key', key_cache', value_cache')``.

    query/key/value [T, H, D] float32 holding model-dtype values; positions and
    slot_mapping [T] ints; cos_sin_cache [P, rotary_dim] float32 (model-dtype
    values); caches [pages, P, Hkv, D] (P-token pages): uint8 codes when ``cache_fp8`` else
    float32 holding model-dtype values."""
    rotary_dim = cos_sin_cache.shape[1]
    cs = np.asarray(cos_sin_cache, dtype=np.float32)[np.asarray(positions)]
    q_out = None if query is None else round_to(rope(query, cs, rotary_dim, is_neox), dtype)
    k_out = round_to(rope(key, cs, rotary_dim, is_neox), dtype)
    v_in = np.asarray(value, dtype=np.float32)
    kc = np.array(key_cache, copy=True)
    vc = np.array(value_cache, copy=True)
    k_store = quantize_rows(k_out, k_scale) if cache_fp8 else k_out
    v_store = quantize_rows(v_in, v_scale) if cache_fp8 else v_in
    page = kc.shape[1]  # tokens per page
    for t, slot in enumerate(np.asarray(slot_mapping)):
        if slot < 0:
            continue
        kc[slot // page, slot % page] = k_store[t]
        vc[slot // page, slot % page] = v_store[t]
    return q_out, k_out, kc, vc
