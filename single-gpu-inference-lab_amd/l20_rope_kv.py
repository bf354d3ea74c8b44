"""Paged KV-cache producer for MI355X: RoPE + (FP8) paged cache write.

Mirrors ``integrations/vllm/l20_rope_kv.py:256-309`` of the reference (paths
relative to its repo root): ``l20_rope_and_cache`` rotates Q and K in place and
writes K and V into the paged NHD caches at ``slot_mapping``, with the same
argument order and error messages.  The reference writes 16-bit caches only
("quantized KV cache is not supported"); here an ``float8_e4m3fn`` cache is
written with the reference quantiser's rule, per-tensor ``k_scale``/``v_scale``
or per-KV-head scale tensors.  ``l20_kv_fp8_scales`` computes those scales
(``max(amax / 448, 1e-12)``) from the values the write would store.

Both call ``torch.ops.l20_stack`` ops of the native library; there is no CPU
fallback.
"""

from __future__ import annotations

from typing import Optional

import torch

import l20_paged_decode  # noqa: F401  (loads the ops library)
from l20_paged_split_kv import is_mi355x


def l20_rope_and_cache(
    query: Optional[torch.Tensor],
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    is_neox: bool,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scale_per_head: Optional[torch.Tensor] = None,
    v_scale_per_head: Optional[torch.Tensor] = None,
) -> None:
    """RoPE on Q (optional) and K in place; K/V written to the paged caches."""
    if not is_mi355x(key.device):
        raise RuntimeError("l20_rope_and_cache requires an MI355X (gfx950) GPU")
    if key.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("l20_rope_and_cache supports FP16 and BF16")
    if value.dtype != key.dtype or (query is not None and query.dtype != key.dtype):
        raise RuntimeError("Q, K, and V must use the same dtype")
    if key_cache.dtype not in (torch.float8_e4m3fn, key.dtype) or value_cache.dtype != key_cache.dtype:
        raise RuntimeError("K/V cache must be torch.float8_e4m3fn or the model dtype")
    if key.ndim != 3 or value.ndim != 3 or (query is not None and query.ndim != 3):
        raise RuntimeError("Q, K, and V must be [tokens, heads, head_dim]")
    if key.shape != value.shape or (query is not None and query.shape[0] != key.shape[0]):
        raise RuntimeError("Q, K, and V shapes are incompatible")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise RuntimeError("cache must use NHD [blocks, block, heads, dim]")
    if key_cache.shape[2:] != key.shape[1:]:
        raise RuntimeError("cache head shape must match K/V")
    if positions.numel() != key.shape[0] or slot_mapping.numel() != key.shape[0]:
        raise RuntimeError("positions and slot_mapping must match token count")
    torch.ops.l20_stack.rope_and_cache(query, key, value, positions, cos_sin_cache, bool(is_neox), key_cache,
                                       value_cache, slot_mapping, float(k_scale), float(v_scale),
                                       k_scale_per_head, v_scale_per_head)


def l20_kv_fp8_scales(
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    is_neox: bool,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    per_head: bool = True,
) -> tuple:
    """fp32 ``(k_scales, v_scales)`` [num_kv_heads] for an fp8 cache: per head, or the
    per-tensor scale repeated in every entry."""
    if not is_mi355x(key.device):
        raise RuntimeError("l20_kv_fp8_scales requires an MI355X (gfx950) GPU")
    ks = torch.empty(key.shape[1], dtype=torch.float32, device=key.device)
    vs = torch.empty_like(ks)
    torch.ops.l20_stack.kv_fp8_scales(key, value, positions, cos_sin_cache, bool(is_neox), key_cache, value_cache,
                                      slot_mapping, ks, vs, bool(per_head))
    return ks, vs
