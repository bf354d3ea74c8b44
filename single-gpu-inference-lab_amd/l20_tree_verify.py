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
  (and the contiguous-cache ``hybrid_tree_attention`` / ``hybrid_tree_attention_split``,
  which view or copy the K/V into 16-token pages first) -- the reference's signatures, with the drafts' K/V in separate contiguous
  ``[B, S, Hkv, D]`` tensors next to a paged prefix of ``cached_length``
  tokens.  The prefix pass (the HBM-bound part) runs on the HIP kernel with
  every draft row a query column and returns its LSE; ``l20_pd_tree_suffix_merge``
  (one more launch) attends each row over its visible drafts and merges the
  two in fp32.  Rows beyond the kernel's 32-column tile are packed as extra
  batch entries that share the sequence's pages.  A ``TreeAttentionWorkspace``
  keeps every buffer between calls, so warmed calls allocate nothing.

The caches are fp8 e4m3fn (with ``k_scale``/``v_scale``) or the query's 16-bit
dtype; head_dim 64 or 128; 16-token pages.
"""

from __future__ import annotations

import math
import weakref
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


def should_use_l20_split_tree_attention(cached_length: int) -> bool:
    """The reference's gate between its monolithic and split (prefix summary +
    suffix summary + merge) tree kernels (``triton_tree_attention.py:1200-1202``,
    True from 4096 cached tokens on L20).  The MI355X path has only the split
    form -- the prefix pass on the streaming kernel, the suffix and merge in one
    more launch -- so it is used for every length."""
    del cached_length
    return True


def l20_tree_attention_block_t(cached_length: int) -> int:
    """The reference's Triton tile policy (``triton_tree_attention.py:1205-1207``):
    128 from 4096 cached tokens, else 64.  The HIP kernels' tiling is fixed; the
    entry points accept and validate ``block_t`` for call compatibility."""
    return 128 if cached_length >= 4096 else 64


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
                tree_words: torch.Tensor, output: torch.Tensor, lse: Optional[torch.Tensor],
                partials=None) -> torch.Tensor:
    """One launch of the split-KV kernel in tree mode over ``rows_q`` [B*q_len, Hq, D];
    ``partials`` (output, max, sum) is the split workspace (allocated when None)."""
    batch = rows_q.shape[0] // q_len
    num_q_heads, head_dim = rows_q.shape[1], rows_q.shape[2]
    if split_size is None:
        split_size = default_split_size(batch, key_cache.shape[2], max_seq_len, rows_q.device)
    if partials is None:
        n_s = max(1, math.ceil(max_seq_len / split_size)) if max_seq_len > 0 else 1
        shape = (rows_q.shape[0], num_q_heads, n_s)
        partials = (torch.empty((*shape, head_dim), device=rows_q.device, dtype=torch.float32),
                    torch.empty(shape, device=rows_q.device, dtype=torch.float32),
                    torch.empty(shape, device=rows_q.device, dtype=torch.float32))
    po, pm, ps = partials
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
        raise ValueError("expected key/value cache=[pages,page,Hkv,D]")
    page = key_cache.shape[1]
    if page < 16 or page % 16 or page > 4096 or (
            page > 16 and any(c.stride(0) != page * c.stride(1) for c in (key_cache, value_cache))):
        raise ValueError("paged tree attention requires pages of a multiple of 16 tokens, held contiguously")
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


class TreeAttentionWorkspace(tuple):
    """The reference's six summary tensors (``triton_tree_attention.py:761-776``:
    output fp32 [B, S, Hq, D], max and sum fp32 [B, S, Hq], for the prefix then
    the suffix), which unpack as a tuple, plus the buffers the MI355X path
    needs: created by the first call that uses them and reused by every later
    call of the same shapes, so a warmed workspace makes
    ``hybrid_tree_attention_paged_prefix`` allocate nothing (and lets it be
    captured in a HIP graph)."""

    def __new__(cls, tensors):
        obj = super().__new__(cls, tensors)
        obj._buffers = {}
        return obj

    def buffer(self, name: str, shape, dtype: torch.dtype, device) -> torch.Tensor:
        shape = tuple(int(x) for x in shape)
        t = self._buffers.get(name)
        if t is None or tuple(t.shape) != shape or t.dtype != dtype or t.device != torch.device(device):
            t = torch.empty(shape, dtype=dtype, device=device)
            self._buffers[name] = t
        return t

    def constant(self, name: str, make, shape, device) -> torch.Tensor:
        """A tensor made once by ``make()`` and kept while its shape and device stay."""
        t = self._buffers.get(name)
        if t is None or tuple(t.shape) != tuple(shape) or t.device != torch.device(device):
            t = make()
            self._buffers[name] = t
        return t


def allocate_tree_attention_workspace(query: torch.Tensor) -> TreeAttentionWorkspace:
    """Workspace of the split tree attention (the reference's six-tensor layout,
    ``triton_tree_attention.py:761-776``); see ``TreeAttentionWorkspace``."""
    if query.ndim != 4:
        raise ValueError("expected query=[B,S,Hq,D]")
    batch, draft_length, num_q_heads, head_dim = query.shape
    summary = (batch, draft_length, num_q_heads)
    f32 = dict(device=query.device, dtype=torch.float32)
    return TreeAttentionWorkspace(
        (torch.empty((*summary, head_dim), **f32), torch.empty(summary, **f32), torch.empty(summary, **f32),
         torch.empty((*summary, head_dim), **f32), torch.empty(summary, **f32), torch.empty(summary, **f32)))


# Six-tensor tuples given as workspaces keep the extra buffers of their wrapper
# across calls: id of the first tensor -> (weak reference to it, the buffer
# dict).  Only the buffers are held, never the caller's tensors, and the entry
# goes when that tensor does.
_WRAPPED = {}


def _as_workspace(workspace, query: torch.Tensor) -> TreeAttentionWorkspace:
    """``workspace`` as a TreeAttentionWorkspace: None allocates one, a
    TreeAttentionWorkspace is used as is, the reference's six-tensor tuple
    (``triton_tree_attention.py:761-776``) is wrapped; anything else is refused
    rather than silently replaced by a fresh allocation."""
    if workspace is None:
        return allocate_tree_attention_workspace(query)
    if isinstance(workspace, TreeAttentionWorkspace):
        return workspace
    if isinstance(workspace, (tuple, list)) and len(workspace) == 6 and all(
            isinstance(t, torch.Tensor) for t in workspace):
        first = workspace[0]
        entry = _WRAPPED.get(id(first))
        if entry is None or entry[0]() is not first:
            entry = (weakref.ref(first), {})
            _WRAPPED[id(first)] = entry
            weakref.finalize(first, _WRAPPED.pop, id(first), None)
        ws = TreeAttentionWorkspace(tuple(workspace))
        ws._buffers = entry[1]
        return ws
    raise TypeError("workspace must come from allocate_tree_attention_workspace (or be its six-tensor tuple)")


def _check_block_t(block_t: Optional[int]) -> None:
    # The reference's Triton tile knob (triton_tree_attention.py:1071-1074); the
    # HIP kernel's tiling is fixed, so it is only validated.
    if block_t is not None and block_t not in (32, 64, 128):
        raise ValueError("block_t must be one of 32, 64, or 128")


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
    block_t: Optional[int] = None,
    contiguous_pages: bool = False,
    page_base: Optional[torch.Tensor] = None,
    k_scale: Scale = 1.0,
    v_scale: Scale = 1.0,
    split_size: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Tree attention over a paged prefix of ``cached_length`` tokens plus a contiguous
    draft suffix (``triton_tree_attention.py:1040-1197``).

    query [B, S, Hq, D]; key/value_cache [pages, P, Hkv, D] (P a multiple of 16);
    suffix_key/value [B, S, Hkv, D] (query dtype); block_table [B, pages] covering
    cached_length (with ``contiguous_pages`` the pages of sequence b are
    ``page_base[b] + t // P`` instead, as in the reference); ancestor_mask [S, S] bool
    on the query's device.  Returns [B, S, Hq, D] in the query dtype (``output`` when
    given).  ``workspace`` is one from ``allocate_tree_attention_workspace`` or the
    reference's six-tensor tuple (wrapped once and kept with the tuple).

    Precision: the prefix pass writes its normalised output in the query dtype
    (the decode op's output type) before the fp32 LSE merge with the suffix, so
    the prefix share of each row is rounded twice (query dtype, then the final
    output): at most one extra half-ulp of bf16 (2^-9 relative) on that share.

    Two launches of the HIP library: the prefix pass (the split-KV kernel with every
    draft row a query column, LSE out) and ``l20_pd_tree_suffix_merge`` (suffix
    attention and LSE merge in fp32).  With a ``TreeAttentionWorkspace`` from
    ``allocate_tree_attention_workspace`` and an ``output`` tensor, a call after the
    first of the same shapes allocates nothing; float (or [Hkv] tensor) scales keep
    it free of host synchronisation.
    """
    _check_common(query, key_cache, value_cache)
    if query.ndim != 4:
        raise ValueError("expected query=[B,S,Hq,D]")
    if suffix_key.ndim != 4 or suffix_value.shape != suffix_key.shape:
        raise ValueError("expected suffix key/value=[B,S,Hkv,D]")
    if block_table.ndim != 2:
        raise ValueError("expected block_table=[B,pages]")
    batch, draft, num_q_heads, head_dim = query.shape
    num_kv_heads = key_cache.shape[2]
    if suffix_key.shape != (batch, draft, num_kv_heads, head_dim):
        raise ValueError("suffix KV must match query batch/draft and cache kv heads")
    if suffix_key.dtype != query.dtype or suffix_value.dtype != query.dtype:
        raise ValueError("suffix key/value must have the query's dtype")
    page = key_cache.shape[1]  # tokens per page (a multiple of 16)
    if block_table.shape[0] != batch or block_table.shape[1] * page < cached_length:
        raise ValueError("block_table does not cover cached_length")
    if ancestor_mask.shape != (draft, draft):
        raise ValueError("ancestor_mask must match draft_length")
    if draft < 1 or draft > MAX_DRAFT:
        raise ValueError("paged suffix path supports draft_length in [1, 64]")
    _check_block_t(block_t)
    if contiguous_pages:
        if page_base is None:
            raise ValueError("contiguous_pages=True requires page_base=[B]")
        if page_base.ndim != 1 or page_base.shape[0] != batch:
            raise ValueError("page_base must have shape [B]")
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    ws = _as_workspace(workspace, query)
    dev = query.device
    if output is None:
        output = torch.empty_like(query)
    elif output.shape != query.shape or output.dtype != query.dtype:
        raise ValueError("output must be shaped like the query, in its dtype")

    # Prefix pass: every draft row sees all cached_length keys.  Rows are packed c at
    # a time (c x group <= 32 query columns) as extra batch entries on the same pages.
    group = num_q_heads // num_kv_heads
    cols = max(1, min(draft, MAX_COLUMNS // group, 32))
    chunks = math.ceil(draft / cols)
    padded = chunks * cols
    entries = batch * chunks
    if padded == draft and query.is_contiguous():
        rows_q = query.view(entries * cols, num_q_heads, head_dim)
    else:
        qb = ws.buffer("query", (batch, padded, num_q_heads, head_dim), query.dtype, dev)
        qb[:, :draft].copy_(query)
        if padded != draft:
            qb[:, draft:].zero_()
        rows_q = qb.view(entries * cols, num_q_heads, head_dim)
    pages = max(1, math.ceil(cached_length / page))
    if contiguous_pages:
        ramp = ws.constant("ramp", lambda: torch.arange(pages, dtype=torch.int32, device=dev), (pages,), dev)
        table = ws.buffer("table", (entries, pages), torch.int32, dev)
        torch.add(page_base.to(torch.int32)[:, None, None], ramp[None, None, :], out=table.view(batch, chunks, pages))
    elif chunks > 1:
        table = ws.buffer("table", (entries, block_table.shape[1]), torch.int32, dev)
        table.view(batch, chunks, -1).copy_(block_table[:, None, :].expand(batch, chunks, block_table.shape[1]))
    else:
        table = block_table
    lens = ws.buffer("lens", (entries,), torch.int32, dev)
    lens.fill_(int(cached_length))
    words = ws.buffer("words", (cols,), torch.int32, dev)
    words.fill_(-1 if cols == 32 else (1 << cols) - 1)
    if split_size is None:
        split_size = default_split_size(entries, num_kv_heads, int(cached_length), dev)
    n_s = max(1, math.ceil(cached_length / split_size)) if cached_length > 0 else 1
    n_rows = entries * cols
    partials = (ws.buffer("partial_output", (n_rows, num_q_heads, n_s, head_dim), torch.float32, dev),
                ws.buffer("partial_max", (n_rows, num_q_heads, n_s), torch.float32, dev),
                ws.buffer("partial_sum", (n_rows, num_q_heads, n_s), torch.float32, dev))
    p_out = ws.buffer("prefix_output", (n_rows, num_q_heads, head_dim), query.dtype, dev)
    p_lse = ws.buffer("prefix_lse", (n_rows, num_q_heads), torch.float32, dev)
    _paged_call(rows_q, key_cache, value_cache, table, lens, cols, int(cached_length), split_size,
                scale, k_scale, v_scale, words, p_out, p_lse, partials=partials)

    # Suffix attention and LSE merge in one launch.
    torch.ops.l20_stack.tree_suffix_merge(
        query, suffix_key, suffix_value, ancestor_mask,
        p_out.view(batch, padded, num_q_heads, head_dim)[:, :draft],
        p_lse.view(batch, padded, num_q_heads)[:, :draft], output, scale)
    return output


def causal_verifier_attention_paged(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    suffix_key: torch.Tensor,
    suffix_value: torch.Tensor,
    block_table: torch.Tensor,
    cached_length: int,
    *,
    block_t: Optional[int] = None,
    workspace=None,
    k_scale: Scale = 1.0,
    v_scale: Scale = 1.0,
    split_size: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """The chain special case (``triton_tree_attention.py:966-1037``): draft row i sees
    the cached prefix and drafts 0..i.  The chain mask is kept in the workspace."""
    if query.ndim != 4:
        raise ValueError("expected query=[B,S,Hq,D]")
    draft = query.shape[1]
    if draft < 1 or draft > MAX_DRAFT:
        raise ValueError("causal verifier path supports draft_length in [1, 64]")
    ws = _as_workspace(workspace, query)
    chain = ws.constant("chain_mask", lambda: make_chain_tree_mask(draft, device=query.device), (draft, draft),
                        query.device)
    return hybrid_tree_attention_paged_prefix(
        query, key_cache, value_cache, suffix_key, suffix_value, block_table, chain, cached_length,
        workspace=ws, block_t=block_t, k_scale=k_scale, v_scale=v_scale, split_size=split_size,
        softmax_scale=softmax_scale, output=output)


def _validate_contiguous(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, ancestor_mask: torch.Tensor,
                         cached_length: int) -> None:
    """The reference's checks of the contiguous-cache entry points
    (``triton_tree_attention.py:683-703``), head_dim 64 also allowed."""
    if query.ndim != 4 or key.ndim != 4 or value.shape != key.shape:
        raise ValueError("expected query=[B,S,Hq,D], key/value=[B,T,Hkv,D]")
    if ancestor_mask.ndim != 2:
        raise ValueError("expected ancestor_mask=[S,S]")
    batch, draft_length, num_q_heads, head_dim = query.shape
    key_batch, total_length, num_kv_heads, key_dim = key.shape
    if key_batch != batch or key_dim != head_dim:
        raise ValueError("query and KV dimensions do not match")
    if total_length != cached_length + draft_length:
        raise ValueError("KV length must equal cached_length + draft_length")
    if ancestor_mask.shape != (draft_length, draft_length):
        raise ValueError("ancestor_mask must match draft_length")
    if head_dim not in (64, 128):
        raise ValueError("head_dim must be 64 or 128")
    if num_q_heads % num_kv_heads:
        raise ValueError("requires an integral GQA ratio")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("key/value must have the query's dtype (fp16 or bf16)")


def _as_pages(x: torch.Tensor, ws: TreeAttentionWorkspace, name: str) -> torch.Tensor:
    """[B, T, H, D] as a [B * ceil(T / 16), 16, H, D] page pool (sequence b on pages
    b * ceil(T / 16) ...): a view when x is contiguous and T is a multiple of 16,
    else a copy into a workspace buffer.  Tokens past a sequence's length in its
    last page (the copy's unwritten tail, or the view's suffix tokens during the
    prefix pass) are loaded but masked: score -inf, V zeroed."""
    batch, total, heads, dim = x.shape
    pages = -(-total // 16)
    if x.is_contiguous() and total % 16 == 0:
        return x.view(batch * pages, 16, heads, dim)
    buf = ws.buffer(name, (batch * pages, 16, heads, dim), x.dtype, x.device)
    buf.view(batch, pages * 16, heads, dim)[:, :total].copy_(x)
    return buf


def _contiguous_tree(query, key, value, ancestor_mask, cached_length, ws, block_t, softmax_scale, output):
    _validate_contiguous(query, key, value, ancestor_mask, cached_length)
    batch, total = key.shape[0], key.shape[1]
    pages = -(-total // 16)
    kp = _as_pages(key, ws, "key_pages")
    vp = _as_pages(value, ws, "value_pages")
    table = ws.constant("contiguous_table",
                        lambda: torch.arange(batch * pages, dtype=torch.int32, device=query.device).view(batch, pages),
                        (batch, pages), query.device)
    return hybrid_tree_attention_paged_prefix(
        query, kp, vp, key[:, cached_length:], value[:, cached_length:], table, ancestor_mask, cached_length,
        workspace=ws, block_t=block_t, softmax_scale=softmax_scale, output=output)


def hybrid_tree_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, ancestor_mask: torch.Tensor,
                          cached_length: int, *, block_t: Optional[int] = None,
                          softmax_scale: Optional[float] = None) -> torch.Tensor:
    """Tree attention over contiguous K/V [B, cached_length + S, Hkv, D] (the
    reference's ``hybrid_tree_attention``, ``triton_tree_attention.py:706-758``):
    every draft row sees the cached prefix, draft j iff ``ancestor_mask[i, j]``.
    Runs the paged path: the prefix as 16-token pages of the same memory, the
    last S tokens as the suffix."""
    _check_block_t(block_t)
    return _contiguous_tree(query, key, value, ancestor_mask, cached_length,
                            allocate_tree_attention_workspace(query), block_t, softmax_scale, None)


def hybrid_tree_attention_split(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                ancestor_mask: torch.Tensor, cached_length: int, *, workspace=None,
                                block_t: Optional[int] = None, softmax_scale: Optional[float] = None,
                                output: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's prefix/suffix-summary form (``triton_tree_attention.py:779-886``)
    of ``hybrid_tree_attention``; a ``TreeAttentionWorkspace`` keeps its buffers
    between calls."""
    _check_block_t(block_t)
    ws = _as_workspace(workspace, query)
    return _contiguous_tree(query, key, value, ancestor_mask, cached_length, ws, block_t, softmax_scale, output)
