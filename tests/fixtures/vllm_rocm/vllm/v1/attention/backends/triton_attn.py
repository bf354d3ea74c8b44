"""Stand-in for the region of vLLM's v1 Triton attention backend
(vllm/v1/attention/backends/triton_attn.py) that the ROCm install hook patches:
the forward's call to ``unified_attention`` over the NHD paged cache.

Not vLLM code: a minimal module with the same call site, variable names and
indentation, so the installer can be exercised (and the patched forward run)
without vLLM installed.  ``unified_attention`` here records its call and
fills the output with -1.
"""

import torch

CALLS = []


def unified_attention(**kwargs):
    CALLS.append(kwargs)
    kwargs["out"].fill_(-1.0)


class TritonAttentionImpl:

    def __init__(self, num_heads, head_size, scale, num_kv_heads, kv_cache_dtype="fp8"):
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.fp8_dtype = torch.float8_e4m3fn
        self.alibi_slopes = None
        self.sliding_window = (-1, -1)
        self.logits_soft_cap = 0
        self.sinks = None

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None):
        num_actual_tokens = attn_metadata.num_actual_tokens
        key_cache, value_cache = kv_cache.unbind(0)
        if self.kv_cache_dtype.startswith("fp8"):
            key_cache = key_cache.view(self.fp8_dtype)
            value_cache = value_cache.view(self.fp8_dtype)

        cu_seqlens_q = attn_metadata.query_start_loc
        seqused_k = attn_metadata.seq_lens
        max_seqlen_q = attn_metadata.max_query_len
        max_seqlen_k = attn_metadata.max_seq_len
        block_table = attn_metadata.block_table

        unified_attention(
            q=query[:num_actual_tokens],
            k=key_cache,
            v=value_cache,
            out=output[:num_actual_tokens],
            cu_seqlens_q=cu_seqlens_q,
            max_seqlen_q=max_seqlen_q,
            seqused_k=seqused_k,
            max_seqlen_k=max_seqlen_k,
            softmax_scale=self.scale,
            causal=True,
            block_table=block_table,
        )
        return output
