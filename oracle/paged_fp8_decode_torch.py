"""CPU torch restatement of the dequantise-then-attend oracle (the CPU baseline).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module: it is the reported CPU baseline (timed on
the GPU box's host cores) and is pinned against the numpy oracle
``paged_fp8_decode_ref.reference`` in ``tests/test_oracle_torch.py``.  The
product path never calls it.

It follows the reference's oracle ``scripts/smoke_cuda_paged_fp8_decode_op.py:22-41``
(paths relative to the reference repo root) step by step, on the CPU and in
fp32 throughout: per sequence, gather ``block_table[b, t // 16]`` / ``t % 16``,
dequantise ``code.float() * scale`` (per tensor or per KV head), attend every
query head to its KV head (``kv_head = q_head // G``), softmax of
``q . k * softmax_scale``, probability-weighted V, and the natural-log LSE.
Unlike the reference's oracle it keeps the dequantised K/V in fp32 (the
reference rounds them to fp16; both agree within the output tolerances, which
``tests/test_oracle.py`` pins), batches the GQA group as a matrix product
instead of ``repeat_interleave``, and handles ``q_len > 1`` with the causal
rule of ``src/l20_stack/ops/triton_tree_attention.py:646`` or explicit
ancestor words (``tree_bits``), and 16-bit caches (scale 1).
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

PAGE_SIZE = 16
Scale = Union[float, torch.Tensor]


def _visible(length: int, q_len: int, tree_bits: Optional[torch.Tensor]) -> torch.Tensor:
    """bool [q_len, length]: row i sees keys before ``length - q_len`` and draft
    key j when j <= i (causal) or bit j of its ancestor word is set."""
    t = torch.arange(length)
    first = length - q_len
    rows = []
    for i in range(q_len):
        if tree_bits is None:
            rows.append(t <= first + i)
        else:
            word = int(tree_bits[i]) & 0xFFFFFFFF
            j = t - first
            drafts = (j >= 0) & (((word >> j.clamp(min=0, max=31)) & 1) == 1)
            rows.append((t < first) | drafts)
    return torch.stack(rows)


def _scaled(codes: torch.Tensor, scale: Scale) -> torch.Tensor:
    """fp32 values of gathered cache rows [L, Hkv, D]."""
    x = codes.float()
    if isinstance(scale, torch.Tensor) and scale.numel() > 1:
        return x * scale.float().view(1, -1, 1)
    return x * float(scale)


def reference_torch(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    block_table: torch.Tensor, seq_lens: torch.Tensor, k_scale: Scale, v_scale: Scale, *,
                    softmax_scale: Optional[float] = None, q_len: int = 1,
                    tree_mask: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(out [B*q_len, Hq, D] fp32, lse [B*q_len, Hq] fp32)`` on the CPU.

    query [B*q_len, Hq, D] (any float dtype); key/value caches [P, 16, Hkv, D]
    float8_e4m3fn (or fp16/bf16 with scale 1); block_table [B, max_pages] int;
    seq_lens [B] int; k/v_scale float or fp32 [Hkv]; tree_mask [B, q_len] int
    ancestor words or None.  Rows with no visible key give zeros and -inf.
    """
    rows, hq, d = query.shape
    batch = rows // q_len
    hkv = key_cache.shape[2]
    group = hq // hkv
    scale = d ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = torch.zeros(rows, hq, d, dtype=torch.float32)
    lse = torch.full((rows, hq), float("-inf"), dtype=torch.float32)
    q_all = query.float()
    for b in range(batch):
        length = int(seq_lens[b])
        if length <= 0:
            continue
        t = torch.arange(length)
        page = key_cache.shape[1]  # tokens per page
        pages = block_table[b].long()[t // page]
        keys = _scaled(key_cache[pages, t % page], k_scale)      # [L, Hkv, D]
        values = _scaled(value_cache[pages, t % page], v_scale)  # [L, Hkv, D]
        # [Hkv, q_len * G, D]: query row i, head kvh * G + g
        q = q_all[b * q_len:(b + 1) * q_len].view(q_len, hkv, group, d).permute(1, 0, 2, 3).reshape(
            hkv, q_len * group, d)
        scores = torch.matmul(q, keys.permute(1, 2, 0)) * scale  # [Hkv, q_len * G, L]
        vis = _visible(length, q_len, None if tree_mask is None else tree_mask[b])  # [q_len, L]
        scores = scores.masked_fill(~vis.repeat_interleave(group, dim=0).unsqueeze(0), float("-inf"))
        row_lse = torch.logsumexp(scores, dim=-1)  # [Hkv, q_len * G]
        probs = torch.exp(scores - row_lse.unsqueeze(-1).clamp(min=-3.0e38))
        attended = torch.matmul(probs, values.permute(1, 0, 2))  # [Hkv, q_len * G, D]
        o = attended.view(hkv, q_len, group, d).permute(1, 0, 2, 3).reshape(q_len, hq, d)
        out[b * q_len:(b + 1) * q_len] = torch.nan_to_num(o, nan=0.0)
        lse[b * q_len:(b + 1) * q_len] = row_lse.view(hkv, q_len, group).permute(1, 0, 2).reshape(q_len, hq)
    return out, lse
