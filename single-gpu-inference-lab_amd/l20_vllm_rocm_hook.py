"""Gated dispatch of vLLM's ROCm decode attention to the MI355X paged FP8 op.

The counterpart of the decode branch that the reference injects into vLLM's
CUDA FlashInfer backend (``integrations/vllm/install_l20_fp8_paged_decode.py:63-149``,
paths relative to the reference repo root).  On ROCm the NHD paged cache
(``[num_blocks, block_size, num_kv_heads, head_size]``) lives in vLLM's Triton attention
backend (``vllm/v1/attention/backends/triton_attn.py``), whose forward calls
``unified_attention`` for every token; ``install_l20_fp8_paged_decode_rocm.py``
inserts, right before that call::

    if l20_fp8_paged_decode_or_none(self, layer, query, key_cache, value_cache,
                                    output, attn_metadata, num_actual_tokens):
        return output

``l20_fp8_paged_decode_or_none`` returns False -- and vLLM runs its own kernel --
unless every gate passes; the gates and their environment variables are the
reference's:

* ``VLLM_ENABLE_L20_FP8_PAGED_DECODE=1`` turns the path on (off by default);
* the device is an MI355X (gfx950; the reference required SM89), no graph is
  being captured, the KV cache is fp8 (``kv_cache_dtype`` "fp8"/"fp8_e4m3" for
  OCP e4m3fn bytes or "fp8_e5m2" for e5m2 bytes -- the reference's hook takes every
  quantized cache, and vLLM's backend views both as its platform fp8 type, so the
  op gets the bytes re-viewed in the setting's format) in blocks of any
  multiple of 16 tokens (vLLM's block size passes through) with head_size 64/128, the batch is pure decode (``max_query_len == 1``)
  and the layer uses none of ALiBi, sliding windows, logit soft-capping,
  attention sinks or a fused output quantisation (``output_scale`` given, or an
  output buffer whose dtype is not the query's);
* ``should_use_l20_paged_fp8_split_kv(batch, max_seq_len)`` agrees, unless
  ``VLLM_L20_FP8_PAGED_FORCE=1``;
* ``VLLM_L20_FP8_PAGED_TRACE=<path>`` appends one JSON line per dispatched call
  (``event``, ``batch``, ``max_seq_len``, ``q_heads``, ``kv_heads``).

The split workspace is cached on the attention impl (``_l20_fp8_workspace``)
and reallocated only when the batch, head count or split count changes.
"""

from __future__ import annotations

import json
import os
from typing import Any, Optional

import torch

ENABLE_ENV = "VLLM_ENABLE_L20_FP8_PAGED_DECODE"
FORCE_ENV = "VLLM_L20_FP8_PAGED_FORCE"
TRACE_ENV = "VLLM_L20_FP8_PAGED_TRACE"
SPLIT_SIZE = 512  # the reference hook's split (install_l20_fp8_paged_decode.py:99-121)


def _unsupported_features(impl: Any) -> bool:
    window = getattr(impl, "sliding_window", None)
    if isinstance(window, (tuple, list)):
        window_on = any(w is not None and w >= 0 for w in window)
    else:
        window_on = window is not None and window not in (-1, 0)
    return (
        getattr(impl, "alibi_slopes", None) is not None
        or window_on
        or bool(getattr(impl, "logits_soft_cap", 0) or 0)
        or getattr(impl, "sinks", None) is not None
    )


_FP8_BYTES = (torch.float8_e4m3fn, torch.float8_e5m2, torch.uint8)


def cache_format(impl: Any) -> Optional[torch.dtype]:
    """The torch dtype that the cache bytes hold, from vLLM's ``kv_cache_dtype``
    ("fp8" and "fp8_e4m3": OCP e4m3fn on gfx950; "fp8_e5m2": e5m2), or None for a
    cache this path does not read.  vLLM's Triton backend views every fp8 cache
    as the platform's fp8 type, so the format comes from the setting, not from
    the tensor's dtype."""
    kind = str(getattr(impl, "kv_cache_dtype", ""))
    if kind in ("fp8", "fp8_e4m3"):
        return torch.float8_e4m3fn
    if kind == "fp8_e5m2":
        return torch.float8_e5m2
    return None


def decode_gate(impl: Any, layer: Any, query: torch.Tensor, key_cache: torch.Tensor,
                value_cache: torch.Tensor, attn_metadata: Any, num_actual_tokens: int,
                output: Optional[torch.Tensor] = None, output_scale: Any = None) -> bool:
    """True when the call may take the MI355X path (all gates but the heuristic).

    A fused output quantisation (vLLM passes ``output_scale``, and the output
    buffer is then fp8) or any output dtype other than the query's is left to
    vLLM's kernel: the op writes the query dtype only.
    """
    from l20_paged_split_kv import is_mi355x

    if os.getenv(ENABLE_ENV, "0") != "1":
        return False
    if cache_format(impl) is None:
        return False
    if getattr(attn_metadata, "max_query_len", None) != 1:
        return False
    if _unsupported_features(impl):
        return False
    if output_scale is not None:
        return False
    if output is not None and (output.dtype != query.dtype or output.dim() < 2
                               or output.shape[0] < num_actual_tokens
                               or output[0].numel() != query[0].numel()):
        return False
    if key_cache.dtype not in _FP8_BYTES or value_cache.dtype not in _FP8_BYTES:
        return False
    if key_cache.dim() != 4 or key_cache.shape != value_cache.shape:
        return False
    _, block, kv_heads, head_size = key_cache.shape
    # vLLM's block size passes through: any multiple of 16 tokens whose rows
    # are contiguous within the block (its NHD caches are)
    if block < 16 or block % 16 or block > 4096 or head_size not in (64, 128) or query.dim() != 3 \
            or query.shape[-1] != head_size:
        return False
    if block > 16 and any(c.stride(0) != block * c.stride(1) for c in (key_cache, value_cache)):
        return False
    q_heads = query.shape[1]
    if q_heads % kv_heads or q_heads // kv_heads > 32:
        return False
    if query.shape[0] < num_actual_tokens or attn_metadata.block_table.shape[0] != num_actual_tokens:
        return False
    if not is_mi355x(query.device):
        return False
    if torch.cuda.is_current_stream_capturing():
        return False
    return True


def l20_fp8_paged_decode_or_none(impl: Any, layer: Any, query: torch.Tensor, key_cache: torch.Tensor,
                                 value_cache: torch.Tensor, output: torch.Tensor, attn_metadata: Any,
                                 num_actual_tokens: int, output_scale: Any = None) -> bool:
    """Run the decode attention on the MI355X op and return True, or return False
    (and touch nothing) when a gate rejects the call."""
    if not decode_gate(impl, layer, query, key_cache, value_cache, attn_metadata, num_actual_tokens,
                       output=output, output_scale=output_scale):
        return False
    from l20_paged_split_kv import (
        allocate_l20_paged_split_kv_workspace,
        l20_paged_split_kv_attention_fp8,
        should_use_l20_paged_fp8_split_kv,
    )

    batch = int(num_actual_tokens)
    max_seq_len = int(attn_metadata.max_seq_len)
    if os.getenv(FORCE_ENV, "0") != "1" and not should_use_l20_paged_fp8_split_kv(batch, max_seq_len):
        return False
    q = query[:batch]
    shape = (batch, q.shape[1], (max_seq_len + SPLIT_SIZE - 1) // SPLIT_SIZE, q.dtype)
    if getattr(impl, "_l20_fp8_workspace_shape", None) != shape:
        impl._l20_fp8_workspace = allocate_l20_paged_split_kv_workspace(q, max_seq_len, split_size=SPLIT_SIZE)
        impl._l20_fp8_workspace_shape = shape
    fmt = cache_format(impl)
    l20_paged_split_kv_attention_fp8(
        q, key_cache.view(fmt), value_cache.view(fmt), attn_metadata.block_table[:batch],
        attn_metadata.seq_lens[:batch],
        k_scale=float(layer._k_scale_float), v_scale=float(layer._v_scale_float),
        max_seq_len=max_seq_len, split_size=SPLIT_SIZE, output=output[:batch].view_as(q),
        workspace=impl._l20_fp8_workspace, softmax_scale=float(impl.scale),
    )
    trace_path = os.getenv(TRACE_ENV)
    if trace_path:
        with open(trace_path, "a", encoding="utf-8") as trace_file:
            trace_file.write(json.dumps({
                "event": "l20_fp8_paged_decode_run",
                "batch": batch,
                "max_seq_len": max_seq_len,
                "q_heads": int(q.shape[1]),
                "kv_heads": int(key_cache.shape[2]),
            }, sort_keys=True) + "\n")
    return True
