"""Speculative tree verification over a paged KV cache on the MI355X decode kernel.

Speculative decoding proposes S draft tokens arranged as a tree; verification
runs attention for the S draft queries of every sequence at once.  Draft row
``i`` sees the whole cached prefix plus the draft tokens that are its ancestors
(``ancestor_mask[i, j]``; a chain -- row ``i`` sees drafts ``0..i`` -- is the
plain causal verifier).  The semantics are the reference's
``src/l20_stack/ops/triton_tree_attention.py`` (paths relative to the reference
repo root): ``torch_tree_attention_reference`` (``:1218-1240``) defines the
visibility, ``make_chain_tree_mask`` (``:1210-1215``) the chain,
``hybrid_tree_attention_paged_prefix`` (``:1040-1197``) and
``causal_verifier_attention_paged`` (``:966-1037``) the paged entry points.

Two entry points:

* ``paged_tree_verify_attention`` -- the drafts' K/V are already in the paged
  cache as each sequence's newest S tokens (how a serving engine lays out a
  verify step).  One launch of the streaming split-KV kernel with per-row
  ancestor bitmasks (``tree_mask``): each K/V page is read once per KV head for
  all S x GQA-group query columns.  Requires S x group <= 32 and S <= 32.
* ``hybrid_tree_attention_paged_prefix`` / ``causal_verifier_attention_paged``
  -- the reference's signatures, with the drafts' K/V in separate contiguous
  ``[B, S, Hkv, D]`` tensors next to a paged prefix of ``cached_length``
  tokens.  The prefix pass (the HBM-bound part) runs on the HIP kernel with
  every draft key visible and returns its LSE; the S x S suffix attention and
  the LSE merge are small fp32 torch ops.  Rows beyond the kernel's 32-column
  tile are packed as extra batch entries that share the sequence's pages.

The caches are fp8 e4m3fn (with ``k_scale``/``v_scale``) or the query's 16-bit
dtype; head_dim 64 or 128; 16-token pages.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import torch

import l20_paged_decode  # noqa: F401  (loads the TORCH_LIBRARY extension)
from l20_paged_split_kv import default_split_size, is_mi355x

Scale = Union[float, torch.Tensor]
MAX_COLUMNS = 32  # query columns (draft rows x GQA group) of one kernel work item
MAX_DRAFT = 64  # the reference's paged suffix limit (triton_tree_attention.py:1095-1096)


def make_chain_tree_mask(draft_length: int, *, device=None) -> torch.Tensor:
    """Lower-triangular ancestor mask of a linear draft chain ([S, S] bool)."""
    positions = torch.arange(draft_length, device=device)
    return positions[None, :] <= positions[:, None]


def tree_mask_bits(ancestor_mask: torch.Tensor) -> torch.Tensor:
    """Boolean ancestor mask ``[..., S, S]`` (row i sees draft j) -> int32 bitmasks
    ``[..., S]`` with bit j of word i set iff ``ancestor_mask[..., i, j]``; S <= 32."""
    if ancestor_mask.dim() < 2 or ancestor_mask.shape[-1] != ancestor_mask.shape[-2]:
        raise ValueError("ancestor_mask must be [..., S, S]")
    s = ancestor_mask.shape[-1]
    if s > 32:
        raise ValueError("tree bitmasks hold at most 32 draft tokens")
    weights = torch.ones(s, dtype=torch.int64, device=ancestor_mask.device) << torch.arange(
        s, dtype=torch.int64, device=ancestor_mask.device)
    words = (ancestor_mask.to(torch.bool).to(torch.int64) * weights).sum(-1)
    # two's-complement view of bit 31 so the word fits int32
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32)


def _scale_args(scale: Scale) -> Tuple[float, Optional[torch.Tensor]]:
    if isinstance(scale, torch.Tensor):
        if scale.numel() == 1:
            return float(scale.reshape(()).item()), None
        return 1.0, scale.to(torch.float32).contiguous()
    return float(scale), None


def _paged_call(rows_q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                block_table: torch.Tensor, seq_lens: torch.Tensor, q_len: int, max_seq_len: int,
                split_size: Optional[int], softmax_scale: float, k_scale: Scale, v_scale: Scale,
                tree_words: torch.Tensor, output: torch.Tensor, lse: Optional[torch.Tensor]) -> torch.Tensor:
    """One launch of the split-KV kernel in tree mode over ``rows_q`` [B*q_len, Hq, D]."""
    batch = rows_q.shape[0] // q_len
    num_q_heads, head_dim = rows_q.shape[1], rows_q.shape[2]
    if split_size is None:
        split_size = default_split_size(batch, key_cache.shape[2], max_seq_len, rows_q.device)
    n_s = max(1, math.ceil(max_seq_len / split_size)) if max_seq_len > 0 else 1
    shape = (rows_q.shape[0], num_q_heads, n_s)
    po = torch.empty((*shape, head_dim), device=rows_q.device, dtype=torch.float32)
    pm = torch.empty(shape, device=rows_q.device, dtype=torch.float32)
    ps = torch.empty(shape, device=rows_q.device, dtype=torch.float32)
    if key_cache.dtype == torch.float8_e4m3fn:
        ks, ks_ph = _scale_args(k_scale)
        vs, vs_ph = _scale_args(v_scale)
        return torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
            rows_q, key_cache, value_cache, block_table, seq_lens, po, pm, ps, output, ks, vs,
            int(max_seq_len), int(split_size), float(softmax_scale), ks_ph, vs_ph, int(q_len), lse, tree_words)
    return torch.ops.l20_stack.paged_decode_split_out(
        rows_q, key_cache, value_cache, block_table, seq_lens, po, pm, ps, output, int(max_seq_len),
        int(split_size), float(softmax_scale), int(q_len), lse, tree_words)


def _check_common(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor) -> None:
    if not is_mi355x(query.device):
        raise RuntimeError("requires an MI355X (gfx950) GPU")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("expected key/value cache=[pages,16,Hkv,D]")
    if key_cache.shape[1] != 16:
        raise ValueError("paged tree attention requires page_size=16")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("query must be fp16 or bf16")
    if key_cache.dtype not in (torch.float8_e4m3fn, query.dtype) or value_cache.dtype != key_cache.dtype:
        raise ValueError("key/value cache must be float8_e4m3fn or the query dtype")
    if query.shape[-1] not in (64, 128) or key_cache.shape[-1] != query.shape[-1]:
        raise ValueError("head_dim must be 64 or 128 and match the cache")
    if query.shape[-2] % key_cache.shape[2]:
        raise ValueError("requires an integral GQA ratio")


def paged_tree_verify_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    ancestor_mask: torch.Tensor,
    *,
    k_scale: Scale = 1.0,
    v_scale: Scale = 1.0,
    max_seq_len: Optional[int] = None,
    split_size: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
    lse: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Tree verification with the drafts' K/V already in the paged cache.

    query          [B, S, Hq, D] (or [B*S, Hq, D]) fp16/bf16
    key/value_cache[pages, 16, Hkv, D] float8_e4m3fn or the query dtype
    block_table    [B, max_pages] int32;  seq_lens [B] int32, each including its S drafts
    ancestor_mask  [S, S] or [B, S, S] bool (row i sees draft j), or the int32
                   bitmasks of ``tree_mask_bits`` ([S] or [B, S])
    Returns ``output`` shaped like ``query``; ``lse`` (fp32 [B*S, Hq]) is written when given.
    """
    _check_common(query, key_cache, value_cache)
    batch = block_table.shape[0]
    rows_q = query.reshape(-1, query.shape[-2], query.shape[-1])
    if rows_q.shape[0] % max(batch, 1):
        raise ValueError("query rows must be batch x draft_length")
    draft = rows_q.shape[0] // batch if batch else (query.shape[1] if query.dim() == 4 else 1)
    if ancestor_mask.dtype == torch.int32:
        words = ancestor_mask
    else:
        words = tree_mask_bits(ancestor_mask)
    if words.shape[-1] != draft or words.dim() not in (1, 2) or (words.dim() == 2 and words.shape[0] != batch):
        raise ValueError("ancestor_mask must match draft_length (and batch)")
    if draft > 32 or draft * (query.shape[-2] // key_cache.shape[2]) > MAX_COLUMNS:
        raise ValueError("draft_length x GQA group must be at most 32")
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item()) if seq_lens.numel() else 0
    scale = query.shape[-1] ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = torch.empty_like(rows_q) if output is None else output.view_as(rows_q)
    _paged_call(rows_q.contiguous(), key_cache, value_cache, block_table, seq_lens, draft, max_seq_len,
                split_size, scale, k_scale, v_scale, words.contiguous(), out, lse)
    return out.view_as(query) if output is None else output


def allocate_tree_attention_workspace(query: torch.Tensor):
    """Prefix and suffix summaries of the split tree attention (the reference's
    six-tensor layout, ``triton_tree_attention.py:761-776``): output fp32
    [B, S, Hq, D], max and sum fp32 [B, S, Hq], for the prefix then the suffix.
    Here the max slot holds the natural-log LSE of the part and the sum slot 1."""
    if query.ndim != 4:
        raise ValueError("expected query=[B,S,Hq,D]")
    batch, draft_length, num_q_heads, head_dim = query.shape
    summary = (batch, draft_length, num_q_heads)
    f32 = dict(device=query.device, dtype=torch.float32)
    return (torch.empty((*summary, head_dim), **f32), torch.empty(summary, **f32), torch.empty(summary, **f32),
            torch.empty((*summary, head_dim), **f32), torch.empty(summary, **f32), torch.empty(summary, **f32))


def _suffix_attention(query: torch.Tensor, suffix_key: torch.Tensor, suffix_value: torch.Tensor,
                      visible: torch.Tensor, scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 attention of the S draft rows over the S draft keys: (out [B,S,Hq,D], lse [B,S,Hq])."""
    group = query.shape[2] // suffix_key.shape[2]
    q = query.float().permute(0, 2, 1, 3).contiguous()  # [B, Hq, S, D]
    k = suffix_key.float().repeat_interleave(group, dim=2).permute(0, 2, 3, 1).contiguous()  # [B, Hq, D, S]
    v = suffix_value.float().repeat_interleave(group, dim=2).permute(0, 2, 1, 3).contiguous()  # [B, Hq, S, D]
    scores = torch.matmul(q, k) * scale
    scores = scores.masked_fill(~visible, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)  # [B, Hq, S]
    probs = torch.exp(scores - torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))[..., None])
    out = torch.matmul(probs, v)
    return out.permute(0, 2, 1, 3), lse.permute(0, 2, 1)


def hybrid_tree_attention_paged_prefix(
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
    k_scale: Scale = 1.0,
    v_scale: Scale = 1.0,
    split_size: Optional[int] = None,
    softmax_scale: Optional[float] = None,
) -> torch.Tensor:
    """Tree attention over a paged prefix of ``cached_length`` tokens plus a contiguous
    draft suffix (``triton_tree_attention.py:1040-1197``).

    query [B, S, Hq, D]; key/value_cache [pages, 16, Hkv, D]; suffix_key/value
    [B, S, Hkv, D] (query dtype); block_table [B, pages] covering cached_length;
    ancestor_mask [S, S] bool.  Returns [B, S, Hq, D] in the query dtype.
    """
    _check_common(query, key_cache, value_cache)
    if query.ndim != 4:
        raise ValueError("expected query=[B,S,Hq,D]")
    if suffix_key.ndim != 4 or suffix_value.shape != suffix_key.shape:
        raise ValueError("expected suffix key/value=[B,S,Hkv,D]")
    batch, draft, num_q_heads, head_dim = query.shape
    num_kv_heads = key_cache.shape[2]
    if suffix_key.shape != (batch, draft, num_kv_heads, head_dim):
        raise ValueError("suffix KV must match query batch/draft and cache kv heads")
    if block_table.ndim != 2 or block_table.shape[0] != batch or block_table.shape[1] * 16 < cached_length:
        raise ValueError("block_table does not cover cached_length")
    if ancestor_mask.shape != (draft, draft):
        raise ValueError("ancestor_mask must match draft_length")
    if draft < 1 or draft > MAX_DRAFT:
        raise ValueError("paged suffix path supports draft_length in [1, 64]")
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    if workspace is None:
        workspace = allocate_tree_attention_workspace(query)
    prefix_out, prefix_lse, prefix_one, suffix_out, suffix_lse, suffix_one = workspace

    # Prefix: every draft row sees all cached_length keys.  Rows are packed c at a
    # time (c x group <= 32 query columns) as extra batch entries on the same pages.
    group = num_q_heads // num_kv_heads
    cols = max(1, min(draft, MAX_COLUMNS // group, 32))
    chunks = math.ceil(draft / cols)
    padded = chunks * cols
    q = query
    if padded != draft:
        q = torch.zeros((batch, padded, num_q_heads, head_dim), dtype=query.dtype, device=query.device)
        q[:, :draft] = query
    rows_q = q.reshape(batch * chunks * cols, num_q_heads, head_dim)
    table = block_table.repeat_interleave(chunks, dim=0) if chunks > 1 else block_table
    lens = torch.full((batch * chunks,), int(cached_length), dtype=torch.int32, device=query.device)
    all_visible = torch.full((cols,), -1 if cols == 32 else (1 << cols) - 1, dtype=torch.int32,
                             device=query.device)
    p_out = torch.empty((rows_q.shape[0], num_q_heads, head_dim), dtype=query.dtype, device=query.device)
    p_lse = torch.empty((rows_q.shape[0], num_q_heads), dtype=torch.float32, device=query.device)
    _paged_call(rows_q, key_cache, value_cache, table.contiguous(), lens, cols, int(cached_length), split_size,
                scale, k_scale, v_scale, all_visible, p_out, p_lse)
    prefix_out.copy_(p_out.view(batch, padded, num_q_heads, head_dim)[:, :draft])
    prefix_lse.copy_(p_lse.view(batch, padded, num_q_heads)[:, :draft])
    prefix_one.fill_(1.0)

    visible = ancestor_mask.to(device=query.device, dtype=torch.bool)[None, None]
    s_out, s_lse = _suffix_attention(query, suffix_key, suffix_value, visible, scale)
    suffix_out.copy_(s_out)
    suffix_lse.copy_(s_lse)
    suffix_one.fill_(1.0)

    m = torch.maximum(prefix_lse, suffix_lse)
    w_p = torch.exp(prefix_lse - m)
    w_s = torch.exp(suffix_lse - m)
    out = (w_p[..., None] * prefix_out + w_s[..., None] * suffix_out) / (w_p + w_s)[..., None]
    return out.to(query.dtype)


def causal_verifier_attention_paged(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    suffix_key: torch.Tensor,
    suffix_value: torch.Tensor,
    block_table: torch.Tensor,
    cached_length: int,
    *,
    k_scale: Scale = 1.0,
    v_scale: Scale = 1.0,
    split_size: Optional[int] = None,
    softmax_scale: Optional[float] = None,
) -> torch.Tensor:
    """The chain special case (``triton_tree_attention.py:966-1037``): draft row i sees
    the cached prefix and drafts 0..i."""
    if query.ndim != 4:
        raise ValueError("expected query=[B,S,Hq,D]")
    return hybrid_tree_attention_paged_prefix(
        query, key_cache, value_cache, suffix_key, suffix_value, block_table,
        make_chain_tree_mask(query.shape[1], device=query.device), cached_length,
        k_scale=k_scale, v_scale=v_scale, split_size=split_size, softmax_scale=softmax_scale)
