"""Dispatcher-backed entry points for the MI355X paged decode operators.

Mirrors ``integrations/vllm/l20_paged_decode.py:1-117`` of the reference
(paths relative to its repo root): ``load_library()`` loads
``l20_paged_decode_ops.so`` from beside this file; ``paged_decode_split_out``
(fp16/bf16 caches), ``paged_decode_fp8_e4m3_split_out`` (fp8 caches) and
``paged_decode_split_indices_out`` (16-bit caches, CSR page lists) call the
``torch.ops.l20_stack`` ops of the same names, and ``register_fake`` meta
implementations return ``output`` so the ops trace under FakeTensor /
torch.compile.  Both run at import.

The native library is required: importing this module raises if the built
``.so`` is missing, and the op has no CPU implementation to fall back on.
"""

from __future__ import annotations

from pathlib import Path
from typing import Optional, Union

import torch

_LIB_NAME = "l20_paged_decode_ops.so"
_loaded = False


def library_path() -> Path:
    return Path(__file__).with_name(_LIB_NAME)


def load_library(path: Optional[Union[str, Path]] = None) -> None:
    """Load the TORCH_LIBRARY(l20_stack) extension (idempotent)."""
    global _loaded
    library = Path(path) if path is not None else library_path()
    if not library.exists():
        raise ImportError(
            f"{library} is missing: build it with `python {Path(__file__).with_name('l20_pd_build.py')}`"
        )
    if _loaded and path is None:
        return
    torch.ops.load_library(str(library))
    _loaded = True


def paged_decode_split_out(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    partial_output: torch.Tensor,
    partial_max: torch.Tensor,
    partial_sum: torch.Tensor,
    output: torch.Tensor,
    max_seq_len: int,
    split_size: int,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    lse: Optional[torch.Tensor] = None,
    tree_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Paged split-KV decode attention over fp16 (or bf16) caches; writes and
    returns ``output``.  The first 11 arguments are the reference's
    (``l20_paged_decode.py:20-45``)."""
    return torch.ops.l20_stack.paged_decode_split_out(
        query, key_cache, value_cache, block_table, seq_lens, partial_output, partial_max, partial_sum,
        output, int(max_seq_len), int(split_size), None if softmax_scale is None else float(softmax_scale),
        int(q_len), lse, tree_mask,
    )


def paged_decode_split(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    max_seq_len: int,
    split_size: int,
) -> torch.Tensor:
    """Allocating form of ``paged_decode_split_out`` (the reference extension's
    ``paged_decode_split``, ``l20_paged_decode.cu:511-547``, exported at
    ``l20_paged_decode.cpp:147``): allocates the split workspace for
    ``ceil(max_seq_len / split_size)`` splits, its o-partials in the query's
    dtype as the reference does, and the output, and returns the output.  Every
    call allocates; serving loops use the ``_out`` form with a reused workspace."""
    if query.dim() != 3:
        raise RuntimeError("invalid query")
    batch, heads, dim = query.shape
    splits = max(1, -(-int(max_seq_len) // int(split_size))) if int(split_size) > 0 else 1
    partial_output = torch.empty(batch, heads, splits, dim, device=query.device, dtype=query.dtype)
    partial_max = torch.empty(batch, heads, splits, device=query.device, dtype=torch.float32)
    partial_sum = torch.empty_like(partial_max)
    output = torch.empty_like(query)
    return paged_decode_split_out(query, key_cache, value_cache, block_table, seq_lens, partial_output, partial_max,
                                  partial_sum, output, max_seq_len, split_size)


def paged_decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
) -> torch.Tensor:
    """The reference extension's ``paged_decode`` (``l20_paged_decode.cu:467-494``,
    exported at ``l20_paged_decode.cpp:146``): decode attention over fp16/bf16
    paged caches with no length bound and no workspace argument, returning a
    new output.  The reference runs one workgroup per (sequence, query head) over
    the whole sequence; here the split kernel runs with the library's split size
    for the longest sequence the block table holds (``block_table.size(1)``
    pages of ``key_cache.size(1)`` tokens, known without reading ``seq_lens``
    back from the device)."""
    from l20_paged_split_kv import default_split_size

    if query.dim() != 3 or key_cache.dim() != 4 or block_table.dim() != 2:
        raise RuntimeError("Q must be [B,H,D], caches [pages,page_size,Hkv,D] and the block table [B,pages]")
    max_seq_len = int(block_table.shape[1]) * int(key_cache.shape[1])
    split = default_split_size(int(query.shape[0]), int(key_cache.shape[2]), max(1, max_seq_len), query.device)
    return paged_decode_split(query, key_cache, value_cache, block_table, seq_lens, max_seq_len, split)


def paged_decode_split_indices_out(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    page_indptr: torch.Tensor,
    page_indices: torch.Tensor,
    seq_lens: torch.Tensor,
    partial_output: torch.Tensor,
    partial_max: torch.Tensor,
    partial_sum: torch.Tensor,
    output: torch.Tensor,
    max_seq_len: int,
    split_size: int,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    lse: Optional[torch.Tensor] = None,
    tree_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """The CSR page-list variant (``l20_paged_decode.cu:600-649``): sequence b's
    pages are ``page_indices[page_indptr[b] : page_indptr[b + 1]]``."""
    return torch.ops.l20_stack.paged_decode_split_indices_out(
        query, key_cache, value_cache, page_indptr, page_indices, seq_lens, partial_output, partial_max,
        partial_sum, output, int(max_seq_len), int(split_size),
        None if softmax_scale is None else float(softmax_scale), int(q_len), lse, tree_mask,
    )


def paged_decode_fp8_e4m3_split_out(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    partial_output: torch.Tensor,
    partial_max: torch.Tensor,
    partial_sum: torch.Tensor,
    output: torch.Tensor,
    k_scale: float,
    v_scale: float,
    max_seq_len: int,
    split_size: int,
    softmax_scale: Optional[float] = None,
    k_scale_per_head: Optional[torch.Tensor] = None,
    v_scale_per_head: Optional[torch.Tensor] = None,
    q_len: int = 1,
    lse: Optional[torch.Tensor] = None,
    tree_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Paged FP8 e4m3fn split-KV decode attention; writes and returns ``output``.

    The first 13 arguments are the reference's (``l20_paged_decode.py:48-77``);
    the rest extend it (see the op schema).
    """
    return torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
        query,
        key_cache,
        value_cache,
        block_table,
        seq_lens,
        partial_output,
        partial_max,
        partial_sum,
        output,
        float(k_scale),
        float(v_scale),
        int(max_seq_len),
        int(split_size),
        None if softmax_scale is None else float(softmax_scale),
        k_scale_per_head,
        v_scale_per_head,
        int(q_len),
        lse,
        tree_mask,
    )


def _register_fake() -> None:
    @torch.library.register_fake("l20_stack::paged_decode_split_out")
    def _paged_decode_split_out_fake(query, key_cache, value_cache, block_table, seq_lens, partial_output,
                                     partial_max, partial_sum, output, max_seq_len, split_size,
                                     softmax_scale=None, q_len=1, lse=None, tree_mask=None):
        return output

    @torch.library.register_fake("l20_stack::paged_decode_split_indices_out")
    def _paged_decode_split_indices_out_fake(query, key_cache, value_cache, page_indptr, page_indices, seq_lens,
                                             partial_output, partial_max, partial_sum, output, max_seq_len,
                                             split_size, softmax_scale=None, q_len=1, lse=None, tree_mask=None):
        return output

    @torch.library.register_fake("l20_stack::paged_decode_fp8_e4m3_split_out")
    def _paged_decode_fp8_e4m3_split_out_fake(
        query,
        key_cache,
        value_cache,
        block_table,
        seq_lens,
        partial_output,
        partial_max,
        partial_sum,
        output,
        k_scale,
        v_scale,
        max_seq_len,
        split_size,
        softmax_scale=None,
        k_scale_per_head=None,
        v_scale_per_head=None,
        q_len=1,
        lse=None,
        tree_mask=None,
    ):
        return output

    @torch.library.register_fake("l20_stack::tree_suffix_merge")
    def _tree_suffix_merge_fake(query, suffix_key, suffix_value, ancestor_mask, prefix_output, prefix_lse, output,
                                softmax_scale):
        return None


load_library()
_register_fake()
