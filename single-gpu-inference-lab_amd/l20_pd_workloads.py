"""Seeded paged FP8-KV decode workloads (the five measured configurations).

Input generation follows the reference's smoke/bench scripts
(``scripts/smoke_cuda_paged_fp8_decode_op.py:13-19,71-93``,
``scripts/benchmark_paged_fp8_kv_decode_attention.py:29,83-85``): an N(0,1)
query in bf16, N(0,1) keys/values quantised to OCP e4m3fn with
``scale = max(amax / 448, 1e-12)`` (per tensor, or per KV head), 16-token pages
placed by a seeded random permutation of a page pool.

Tensors are produced on ``device`` with a ``torch.Generator`` seeded per
config, so every consumer that is handed the same tensors (the HIP op, a CPU
checker given ``.cpu()`` copies) sees identical bytes.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, Optional, Union

import torch

FP8_MAX = 448.0
PAGE_SIZE = 16
# The lognormal spread of config 3 is not fixed by its description; this value
# is the one every measurement of it uses.
LOGNORMAL_SIGMA = 1.0


@dataclasses.dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    q_len: int = 1
    context: Optional[int] = None          # fixed length per sequence
    seq_len_range: Optional[tuple] = None  # uniform inclusive [lo, hi]
    lognormal_median: Optional[int] = None
    lognormal_clip: tuple = (16, 8192)
    pool_pages: Optional[int] = None       # explicit pool size
    pool_factor: Optional[float] = None    # pool = ceil(factor * pages needed)
    per_head_scales: bool = False
    softmax_scale: Optional[float] = None
    seed: int = 0

    @property
    def group(self) -> int:
        return self.num_q_heads // self.num_kv_heads


CONFIGS: Dict[str, DecodeConfig] = {
    "c1_qwen2.5_0.5b": DecodeConfig(
        "c1_qwen2.5_0.5b", batch=4, num_q_heads=14, num_kv_heads=2, head_dim=64,
        seq_len_range=(64, 512), pool_pages=256, softmax_scale=1.0 / 8.0, seed=29),
    "c2_qwen2.5_coder_3b": DecodeConfig(
        "c2_qwen2.5_coder_3b", batch=32, num_q_heads=16, num_kv_heads=2, head_dim=128,
        context=2048, pool_pages=8192, per_head_scales=True, seed=31),
    "c3_qwen2.5_7b": DecodeConfig(
        "c3_qwen2.5_7b", batch=128, num_q_heads=28, num_kv_heads=4, head_dim=128,
        lognormal_median=1024, lognormal_clip=(16, 8192), pool_factor=1.2, seed=37),
    "c4_llama3_8b_long": DecodeConfig(
        "c4_llama3_8b_long", batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128,
        context=131072, pool_factor=1.0, per_head_scales=True, seed=41),
    "c5_llama3_70b_verify": DecodeConfig(
        "c5_llama3_70b_verify", batch=64, num_q_heads=64, num_kv_heads=8, head_dim=128,
        q_len=4, context=4096, pool_factor=1.0, seed=43),
}
CONFIG_ORDER = list(CONFIGS)
HEADLINE = "c3_qwen2.5_7b"


def make_seq_lens(cfg: DecodeConfig, gen: torch.Generator) -> torch.Tensor:
    """int32 [B] lengths (each includes the ``q_len`` new tokens)."""
    if cfg.context is not None:
        return torch.full((cfg.batch,), cfg.context, dtype=torch.int32)
    if cfg.seq_len_range is not None:
        lo, hi = cfg.seq_len_range
        return torch.randint(lo, hi + 1, (cfg.batch,), generator=gen, dtype=torch.int64).to(torch.int32)
    if cfg.lognormal_median is not None:
        normal = torch.randn(cfg.batch, generator=gen, dtype=torch.float64)
        raw = torch.exp(math.log(cfg.lognormal_median) + LOGNORMAL_SIGMA * normal)
        lo, hi = cfg.lognormal_clip
        return raw.round().clamp(lo, hi).to(torch.int32)
    raise ValueError(f"config {cfg.name} has no sequence-length rule")


def quantize_fp8_e4m3(x: torch.Tensor, per_head_axis: Optional[int] = None, floor: float = 1.0e-12):
    """OCP e4m3fn quantisation; returns ``(codes, scale)``.

    ``scale`` is a python float (per tensor) or a float32 tensor [Hkv] (per
    head, ``per_head_axis`` = the head axis of ``x``).
    """
    xf = x.float()
    if per_head_axis is None:
        scale = max(float(xf.abs().max()) / FP8_MAX, floor)
        q = (xf / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
        return q, scale
    moved = xf.movedim(per_head_axis, 0)
    amax = moved.reshape(moved.shape[0], -1).abs().amax(dim=1)
    scales = torch.clamp(amax / FP8_MAX, min=floor).to(torch.float32)
    shape = [1] * xf.dim()
    shape[per_head_axis] = -1
    q = (xf / scales.view(shape)).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scales


def _gen(device: Union[str, torch.device], seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_inputs(cfg: DecodeConfig, device: Union[str, torch.device] = "cpu",
                seed: Optional[int] = None, chunk_pages: int = 4096,
                kv_dtype: Optional[torch.dtype] = None) -> dict:
    """Build one seeded input set for ``cfg`` on ``device``.

    Returns a dict with ``query`` [B*q, Hq, D] bf16, ``key_cache`` /
    ``value_cache`` [P, 16, Hkv, D] float8_e4m3fn, ``block_table`` [B, max_pages]
    int32, ``seq_lens`` [B] int32, ``k_scale`` / ``v_scale`` (float or fp32
    [Hkv]), ``softmax_scale``, ``q_len`` and ``max_seq_len``.  With
    ``kv_dtype`` bf16 (or fp16) the caches keep that dtype (the query takes it
    too) and both scales are 1.0.
    """
    seed = cfg.seed if seed is None else seed
    cpu = _gen("cpu", seed)
    seq_lens = make_seq_lens(cfg, cpu)
    pages_per_seq = (seq_lens.to(torch.int64) + PAGE_SIZE - 1) // PAGE_SIZE
    needed = int(pages_per_seq.sum())
    max_pages = int(pages_per_seq.max())
    if cfg.pool_pages is not None:
        pool = cfg.pool_pages
    else:
        pool = int(math.ceil((cfg.pool_factor or 1.0) * needed))
    if pool < needed:
        raise ValueError("page pool smaller than the pages needed")
    perm = torch.randperm(pool, generator=cpu)[:needed].to(torch.int32)
    table = torch.zeros(cfg.batch, max_pages, dtype=torch.int32)
    offset = 0
    for b in range(cfg.batch):
        n = int(pages_per_seq[b])
        table[b, :n] = perm[offset:offset + n]
        offset += n

    dev = torch.device(device)
    g = _gen(dev, seed + 1)
    rows = cfg.batch * cfg.q_len
    q_dtype = kv_dtype if kv_dtype is not None else torch.bfloat16
    query = torch.randn(rows, cfg.num_q_heads, cfg.head_dim, generator=g, device=dev,
                        dtype=torch.float32).to(q_dtype)
    shape = (pool, PAGE_SIZE, cfg.num_kv_heads, cfg.head_dim)
    caches = []
    for _ in range(2):
        # Generate in page chunks so that the fp32 staging stays bounded.
        raw = torch.empty(shape, dtype=q_dtype, device=dev)
        for start in range(0, pool, chunk_pages):
            stop = min(start + chunk_pages, pool)
            raw[start:stop] = torch.randn((stop - start,) + shape[1:], generator=g, device=dev,
                                          dtype=torch.float32).to(q_dtype)
        if kv_dtype is not None:
            caches.append((raw, 1.0))
            continue
        codes, scale = quantize_fp8_e4m3(raw, per_head_axis=2 if cfg.per_head_scales else None)
        del raw
        caches.append((codes, scale))
    (key_cache, k_scale), (value_cache, v_scale) = caches
    softmax_scale = cfg.softmax_scale if cfg.softmax_scale is not None else cfg.head_dim ** -0.5
    return {
        "config": cfg,
        "query": query,
        "key_cache": key_cache,
        "value_cache": value_cache,
        "block_table": table.to(dev),
        "seq_lens": seq_lens.to(dev),
        "k_scale": k_scale,
        "v_scale": v_scale,
        "softmax_scale": float(softmax_scale),
        "q_len": cfg.q_len,
        "max_seq_len": int(seq_lens.max()),
    }


def kv_bytes(seq_lens: torch.Tensor, num_kv_heads: int, head_dim: int, elem_bytes: int = 1) -> int:
    """Algorithmic K+V bytes read per call: ``sum(L) * Hkv * D * 2 * elem_bytes``
    (1 for fp8 caches, 2 for 16-bit ones)."""
    return int(seq_lens.to(torch.int64).sum()) * num_kv_heads * head_dim * 2 * elem_bytes
