"""Opt-in dispatch of tree / causal-verifier attention to the MI355X kernels.

The counterpart of the reference's ``integrations/vllm/l20_tree_attention_dispatch.py``
(paths relative to the reference repo root): the same function names, the same
environment switch (``VLLM_ENABLE_L20_TREE_ATTENTION=1``), the same gates and
cached-length thresholds (4096 tokens for trees, 1024 for the causal verifier
with 2..64 drafts, ``:20-70``), and ``maybe_*`` helpers that return ``None``
whenever a gate rejects the call so the caller runs its own kernel
(``:73-136``).  Differences: the device must be an MI355X (gfx950) instead of
SM89, and head_dim may be 64 as well as 128.  Like the reference, the gates
keep 16-bit caches of the query's dtype (the fp8 paths take scales these
helpers do not pass) and refuse to dispatch while a graph is being captured.
"""

from __future__ import annotations

import os
from typing import Optional

import torch

import l20_tree_verify as tv
from l20_paged_split_kv import is_mi355x

ENABLE_ENV = "VLLM_ENABLE_L20_TREE_ATTENTION"


def l20_tree_attention_enabled() -> bool:
    return os.getenv(ENABLE_ENV, "0") == "1"


def should_dispatch_l20_tree_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    suffix_key: torch.Tensor,
    block_table: torch.Tensor,
    cached_length: int,
    *,
    min_cached_length: int = 4096,
) -> bool:
    if not l20_tree_attention_enabled():
        return False
    if not is_mi355x(query.device):
        return False
    if torch.cuda.is_current_stream_capturing():
        return False
    if query.dtype not in (torch.float16, torch.bfloat16):
        return False
    if key_cache.dtype != query.dtype:
        return False
    if query.ndim != 4 or key_cache.ndim != 4 or suffix_key.ndim != 4:
        return False
    if query.shape[-1] not in (64, 128) or key_cache.shape[-1] != query.shape[-1]:
        return False
    page = key_cache.shape[1]
    if page < 16 or page % 16 or page > 4096:
        return False
    if page > 16 and key_cache.stride(0) != page * key_cache.stride(1):
        return False
    if query.shape[0] != block_table.shape[0]:
        return False
    if query.shape[1] != suffix_key.shape[1]:
        return False
    return cached_length >= min_cached_length


def should_dispatch_l20_causal_verifier_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    suffix_key: torch.Tensor,
    block_table: torch.Tensor,
    cached_length: int,
) -> bool:
    if query.ndim != 4:
        return False
    draft_length = query.shape[1]
    if draft_length < 2 or draft_length > 64:
        return False
    return should_dispatch_l20_tree_attention(query, key_cache, suffix_key, block_table, cached_length,
                                              min_cached_length=1024)


def maybe_l20_tree_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    suffix_key: torch.Tensor,
    suffix_value: torch.Tensor,
    block_table: torch.Tensor,
    ancestor_mask: torch.Tensor,
    cached_length: int,
    *,
    workspace=None,
) -> Optional[torch.Tensor]:
    """Hybrid tree attention on the MI355X path, or ``None`` (run your own kernel)."""
    if not should_dispatch_l20_tree_attention(query, key_cache, suffix_key, block_table, cached_length):
        return None
    if workspace is None:
        workspace = tv.allocate_tree_attention_workspace(query)
    return tv.hybrid_tree_attention_paged_prefix(query, key_cache, value_cache, suffix_key, suffix_value,
                                                 block_table, ancestor_mask, cached_length, workspace=workspace)


def maybe_l20_causal_verifier_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    suffix_key: torch.Tensor,
    suffix_value: torch.Tensor,
    block_table: torch.Tensor,
    cached_length: int,
    *,
    workspace=None,
) -> Optional[torch.Tensor]:
    """The causal (chain) verifier on the MI355X path, or ``None``."""
    if not should_dispatch_l20_causal_verifier_attention(query, key_cache, suffix_key, block_table, cached_length):
        return None
    return tv.causal_verifier_attention_paged(query, key_cache, value_cache, suffix_key, suffix_value, block_table,
                                              cached_length, workspace=workspace)
