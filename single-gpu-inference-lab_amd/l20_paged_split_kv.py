"""Hook-facing paged split-KV FP8 decode attention (MI355X).

Keeps the function names, keyword arguments and error behaviour of the
reference's vLLM-facing module ``integrations/vllm/l20_paged_split_kv.py``
(relative to the reference repo root):

* ``allocate_l20_paged_split_kv_workspace`` (``:14-30``)
* ``l20_paged_split_kv_attention_fp8``     (``:597-695``)
* ``l20_paged_split_kv_attention``         (``:491-595``, fp16/bf16 caches)
* ``should_use_l20_paged_fp8_split_kv``    (``:705-709``)

but runs the hand-written HIP kernels behind
``torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out`` instead of Triton.
Differences: any split size the op accepts (multiple of 16 in [64, 1024]),
no cap on the split count, an fp32 partial workspace with exactly
``ceil(max_seq_len / split_size)`` splits, bf16/fp16 queries, head_dim 64 or
128, per-head scales, ``q_len > 1`` (causal among the new tokens) and an
optional fp32 LSE output.  Caches are float8_e4m3fn or float8_e5m2, as the
reference's dtype check allows (``:617-621``).  Strided K/V views (vLLM's ``kv_cache.unbind(1)``)
are honoured.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import torch

import l20_paged_decode  # noqa: F401  (loads the TORCH_LIBRARY extension)

Workspace = Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]
Scale = Union[float, torch.Tensor]



def _page_ok(key_cache: torch.Tensor, value_cache: torch.Tensor) -> bool:
    """Pages of any multiple of 16 tokens (the reference's Triton path takes any page
    size, ``integrations/vllm/l20_paged_split_kv.py:156,182-200``); above 16 the
    kernels read a page as 16-token sub-pages, so its tokens must be contiguous."""
    page = key_cache.shape[1]
    if page < 16 or page % 16 or page > 4096:
        return False
    return page == 16 or all(c.stride(0) == page * c.stride(1) for c in (key_cache, value_cache))

def _num_splits(max_seq_len: int, split_size: int) -> int:
    return max(1, math.ceil(max_seq_len / split_size)) if max_seq_len > 0 else 1


def is_mi355x(device: Optional[torch.device] = None) -> bool:
    if not torch.cuda.is_available():
        return False
    props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
    return getattr(props, "gcnArchName", "").split(":")[0] == "gfx950"


def allocate_l20_paged_split_kv_workspace(
    query: torch.Tensor,
    max_seq_len: int,
    *,
    split_size: int = 512,
) -> Workspace:
    """``(partial_output fp32 [R,H,n_s,D], partial_max [R,H,n_s], partial_sum [R,H,n_s], output)``.

    ``R`` is ``query.shape[0]`` (batch * q_len) and ``n_s = ceil(max_seq_len / split_size)``.
    """
    rows, num_q_heads, head_dim = query.shape
    num_splits = _num_splits(max_seq_len, split_size)
    partial_shape = (rows, num_q_heads, num_splits)
    return (
        torch.empty((*partial_shape, head_dim), device=query.device, dtype=torch.float32),
        torch.empty(partial_shape, device=query.device, dtype=torch.float32),
        torch.empty(partial_shape, device=query.device, dtype=torch.float32),
        torch.empty_like(query),
    )


def _split_scale(scale: Scale, name: str) -> Tuple[float, Optional[torch.Tensor]]:
    if isinstance(scale, torch.Tensor):
        if scale.numel() == 1:
            return float(scale.reshape(()).item()), None
        return 1.0, scale.to(torch.float32).contiguous()
    return float(scale), None


def l20_paged_split_kv_attention_fp8(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    k_scale: Scale,
    v_scale: Scale,
    max_seq_len: Optional[int] = None,
    split_size: Optional[int] = 512,
    output: Optional[torch.Tensor] = None,
    workspace: Optional[Workspace] = None,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    lse: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Paged FP8 decode attention; returns ``output`` ([B*q_len, Hq, D], query dtype).

    ``k_scale``/``v_scale`` are floats (per tensor) or fp32 tensors of shape
    [Hkv] (per KV head).  ``split_size=None`` lets the library choose.
    """
    if not is_mi355x(query.device):
        raise RuntimeError("requires an MI355X (gfx950) GPU")
    if query.ndim != 3 or key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise RuntimeError("expected Q=[B,H,D], cache=[pages,page,Hkv,D]")
    if key_cache.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2) or value_cache.dtype != key_cache.dtype:
        raise RuntimeError("key/value cache must use a torch FP8 dtype")
    rows, num_q_heads, head_dim = query.shape
    _, page_size, num_kv_heads, cache_dim = key_cache.shape
    batch = rows // q_len if q_len > 0 else -1
    if (
        head_dim not in (64, 128)
        or cache_dim != head_dim
        or not _page_ok(key_cache, value_cache)
        or num_q_heads % num_kv_heads
        or q_len < 1
        or rows % q_len
        or block_table.shape[0] != batch
        or seq_lens.numel() != batch
    ):
        raise RuntimeError("requires compatible head_dim=64/128 GQA tensors with pages of a multiple of 16 tokens")
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item())
    if split_size is None:
        split_size = default_split_size(batch, num_kv_heads, max_seq_len, query.device)
    num_splits = _num_splits(max_seq_len, split_size)
    partial_shape = (rows, num_q_heads, num_splits)
    if workspace is None:
        workspace = allocate_l20_paged_split_kv_workspace(query, max_seq_len, split_size=split_size)
    partial_output, partial_max, partial_sum, workspace_output = workspace
    if output is None:
        output = workspace_output
    if (
        tuple(partial_output.shape[:2]) != partial_shape[:2]
        or partial_output.shape[2] < num_splits
        or partial_output.shape[3] != head_dim
        or tuple(partial_max.shape[:2]) != partial_shape[:2]
        or partial_max.shape[2] < num_splits
        or partial_sum.shape != partial_max.shape
        or output.shape != query.shape
    ):
        raise RuntimeError("paged split-KV workspace shape does not match the request")
    ks, ks_ph = _split_scale(k_scale, "k_scale")
    vs, vs_ph = _split_scale(v_scale, "v_scale")
    return torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
        query, key_cache, value_cache, block_table, seq_lens,
        partial_output, partial_max, partial_sum, output,
        ks, vs, int(max_seq_len), int(split_size),
        softmax_scale, ks_ph, vs_ph, int(q_len), lse,
    )


def l20_paged_split_kv_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    split_size: Optional[int] = 512,
    workspace: Optional[Workspace] = None,
    page_granular: bool = False,
    grouped_gqa: bool = False,
    max_seq_len: Optional[int] = None,
    output: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    lse: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Paged decode attention over fp16/bf16 caches (the query's dtype); returns the
    output ([B*q_len, Hq, D]).  The reference's 16-bit hook-facing function
    (``l20_paged_split_kv.py:491-595``) with its names, keywords and errors,
    running ``torch.ops.l20_stack.paged_decode_split_out``.  ``page_granular``
    and ``grouped_gqa`` choose between the reference's Triton kernel variants;
    the HIP kernel has one form, so they are accepted and change nothing.
    ``max_seq_len`` (default: ``seq_lens.max()``, a host read as in the
    reference), ``output``, ``softmax_scale``, ``q_len`` and ``lse`` are the
    fp8 function's extensions."""
    del page_granular, grouped_gqa
    if not is_mi355x(query.device):
        raise RuntimeError("requires an MI355X (gfx950) GPU")
    if query.ndim != 3 or key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise RuntimeError("expected Q=[B,H,D], cache=[pages,page,Hkv,D]")
    rows, num_q_heads, head_dim = query.shape
    _, page_size, num_kv_heads, cache_dim = key_cache.shape
    batch = rows // q_len if q_len > 0 else -1
    if (
        head_dim not in (64, 128)
        or cache_dim != head_dim
        or not _page_ok(key_cache, value_cache)
        or num_q_heads % num_kv_heads
        or q_len < 1
        or rows % q_len
        or block_table.shape[0] != batch
        or seq_lens.numel() != batch
    ):
        raise RuntimeError("requires compatible head_dim=64/128 GQA tensors with pages of a multiple of 16 tokens")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise RuntimeError("K/V cache must have the query's dtype (fp16 or bf16)")
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item()) if seq_lens.numel() else 0
    if split_size is None:
        split_size = default_split_size(batch, num_kv_heads, max_seq_len, query.device)
    num_splits = _num_splits(max_seq_len, split_size)
    if workspace is None:
        workspace = allocate_l20_paged_split_kv_workspace(query, max_seq_len, split_size=split_size)
    partial_output, partial_max, partial_sum, workspace_output = workspace
    if output is None:
        output = workspace_output
    if (
        tuple(partial_output.shape[:2]) != (rows, num_q_heads)
        or partial_output.shape[2] < num_splits
        or partial_output.shape[3] != head_dim
        or tuple(partial_max.shape[:2]) != (rows, num_q_heads)
        or partial_max.shape[2] < num_splits
        or partial_sum.shape != partial_max.shape
        or output.shape != query.shape
    ):
        raise RuntimeError("paged split-KV workspace shape does not match the request")
    return torch.ops.l20_stack.paged_decode_split_out(
        query, key_cache, value_cache, block_table, seq_lens,
        partial_output, partial_max, partial_sum, output,
        int(max_seq_len), int(split_size), softmax_scale, int(q_len), lse,
    )


def default_split_size(batch: int, num_kv_heads: int, max_seq_len: int,
                       device: Optional[torch.device] = None) -> int:
    """Split size from the library's heuristic for the device's CU count."""
    import l20_pd_cabi

    cus = 256
    if torch.cuda.is_available():
        cus = torch.cuda.get_device_properties(device if device is not None else 0).multi_processor_count
    return int(l20_pd_cabi.load().l20_pd_default_split_size(batch, num_kv_heads, max_seq_len, cus))


def should_use_l20_paged_split_kv(batch: int, max_seq_len: int) -> bool:
    """Heuristic gate of the 16-bit-cache path: closed, as in the reference
    (``l20_paged_split_kv.py:698-702``)."""
    del batch, max_seq_len
    return False


def should_use_l20_paged_fp8_split_kv(batch: int, max_seq_len: int) -> bool:
    """Heuristic dispatch gate used by the vLLM hook: closed for every shape.

    The reference keeps this gate closed (``l20_paged_split_kv.py:705-709``,
    asserted by ``tests/test_l20_paged_split_kv_policy.py:26-43``) because its
    microbenchmark win did not survive a vLLM serving comparison.  No serving
    comparison of the MI355X kernel against vLLM's own ROCm decode kernel
    exists (vLLM is not installed where this was built), so the gate stays
    closed here too; ``VLLM_L20_FP8_PAGED_FORCE=1`` in the hook bypasses it,
    exactly as in the reference hook (``install_l20_fp8_paged_decode.py:63-90``).
    """
    del batch, max_seq_len
    return False
