"""CPU oracle for paged FP8 (OCP e4m3fn, or e5m2) KV-cache decode attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline).  The product path never calls it: the
HIP library fails loudly when it is missing instead of falling back here.

What it restates (reference file:line, relative to the reference repo root):

* ``quantize_fp8_e4m3``  -- ``scripts/smoke_cuda_paged_fp8_decode_op.py:13-19``:
  per-tensor ``scale = max(amax / 448, 1e-12)``, ``clamp(+-448)``, round to
  e4m3fn.  The per-head variant applies the same rule to each KV head.
* ``reference``         -- ``scripts/smoke_cuda_paged_fp8_decode_op.py:22-41``:
  gather ``block_table[b, t // P]`` / ``t % P`` (P-token pages, 16 by default), dequantise in fp32
  (``code * scale``), repeat each KV head over its GQA group, softmax of
  ``q . k * softmax_scale`` and the probability-weighted sum of V.  Extended
  (closed-form, see below) to per-head scales, any softmax scale, head_dim 64,
  ``q_len > 1`` with the causal rule of
  ``src/l20_stack/ops/triton_tree_attention.py:646`` (draft row ``i`` sees
  cached keys plus draft keys ``j <= i``) and an fp32 natural-log LSE.
* ``split_reference``   -- the split-KV partial/merge arithmetic of
  ``integrations/vllm/cuda/l20_paged_decode.cu:291-463`` and
  ``integrations/vllm/l20_paged_split_kv.py:134-239,459-488``: per split the
  running max ``m``, the sum ``l`` of ``exp(s - m)`` and the unnormalised
  output, merged with ``exp(m_s - M)`` corrections.
* ``brute_force_fp64``  -- a scalar float64 loop restatement for tiny inputs.

How each function is pinned (tests/test_oracle.py):

* ``e4m3fn_decode_table``: all 256 codes against the closed form
  ``(-1)^s 2^(e-7) (1 + m/8)`` / ``2^-6 m/8`` and against torch's own
  ``float8_e4m3fn -> float32`` conversion.
* ``e5m2_decode_table``: all 256 codes against torch's ``float8_e5m2 ->
  float32`` conversion and against the top byte of an fp16 (e5m2 is fp16
  with the low 8 mantissa bits dropped: code ``c`` is the fp16 ``c << 8``).
* ``encode_e4m3fn`` / ``quantize_*``: against torch's ``.to(float8_e4m3fn)``
  (round-to-nearest-even) on random values and on every midpoint between
  adjacent codes.
* ``reference``: brute force in float64 loops on tiny shapes; closed forms
  (equal keys give the mean of V, one token gives V_0, equal scores give
  ``LSE = s + ln L``); the reference's own masked-attention KAT
  (``tests/test_tree_attention.py:36-53``) restated with the chain mask;
  invariances (page permutation, GQA replication vs MHA, equal per-head
  scales vs per-tensor, causal row ``i`` vs a ``q_len = 1`` call on the
  shortened sequence).
* ``split_reference``: equal to ``reference`` for every split size.
* ``reference(round_kv_to=np.float16)`` (the reference oracle's literal
  ``(fp8.float() * scale).to(fp16)`` dequantisation,
  ``scripts/smoke_cuda_paged_fp8_decode_op.py:23-24``): bit-equal to the fp32
  path for power-of-two scales (exact in fp16), equal to a torch restatement
  with torch's own fp16 rounding otherwise, and within the output/LSE
  tolerances of the fp32 path on every configuration shape.
* ``reference(acc_dtype=np.float64)``: the float64 brute force to 1e-12.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple, Union

import numpy as np

FP8_E4M3FN_MAX = 448.0
PAGE_SIZE = 16
LOG2E = 1.4426950408889634

ScaleLike = Union[float, Sequence[float], np.ndarray]


# --------------------------------------------------------------------------
# FP8 e4m3fn codec
# --------------------------------------------------------------------------
def e4m3fn_decode_table() -> np.ndarray:
    """float32 value of each of the 256 OCP e4m3fn codes (NaN for 0x7F/0xFF).

    Bit layout s.eeee.mmm, exponent bias 7, no infinities; exponent field 0
    is subnormal ``2^-6 * m / 8``; ``e == 15 and m == 7`` is NaN.
    """
    table = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 3) & 0xF
        mantissa = code & 0x7
        if exponent == 0xF and mantissa == 0x7:
            table[code] = np.nan
        elif exponent == 0:
            table[code] = sign * math.ldexp(mantissa / 8.0, -6)
        else:
            table[code] = sign * math.ldexp(1.0 + mantissa / 8.0, exponent - 7)
    return table


_DECODE = e4m3fn_decode_table()
# Non-negative finite codes 0x00..0x7E are monotonically increasing.
_POSITIVE = _DECODE[:0x7F].astype(np.float64)


def e4m3fn_to_f32(codes: np.ndarray) -> np.ndarray:
    """Decode uint8 e4m3fn codes to float32 (exact)."""
    return _DECODE[np.asarray(codes, dtype=np.uint8)]


def e5m2_decode_table() -> np.ndarray:
    """float32 value of each of the 256 OCP e5m2 codes.

    Bit layout s.eeeee.mm, exponent bias 15, IEEE-style specials: exponent
    field 0 is subnormal ``2^-14 * m / 4``, exponent 31 is +-inf (m == 0) or
    NaN.  The reference's Triton path accepts float8_e5m2 caches and
    dequantises them as ``code.to(float32) * scale``
    (``integrations/vllm/l20_paged_split_kv.py:188-199,617-621``).
    """
    table = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 2) & 0x1F
        mantissa = code & 0x3
        if exponent == 0x1F:
            table[code] = sign * np.inf if mantissa == 0 else np.nan
        elif exponent == 0:
            table[code] = sign * math.ldexp(mantissa / 4.0, -14)
        else:
            table[code] = sign * math.ldexp(1.0 + mantissa / 4.0, exponent - 15)
    return table


_DECODE_E5M2 = e5m2_decode_table()
KV_FORMATS = ("e4m3fn", "e5m2")


def decode_table(kv_format: str = "e4m3fn") -> np.ndarray:
    """The 256-entry decode table of ``kv_format`` ("e4m3fn" or "e5m2")."""
    if kv_format == "e4m3fn":
        return _DECODE
    if kv_format == "e5m2":
        return _DECODE_E5M2
    raise ValueError(f"unknown fp8 format {kv_format!r}")


def fp8_to_f32(codes: np.ndarray, kv_format: str = "e4m3fn") -> np.ndarray:
    """Decode uint8 codes of ``kv_format`` to float32 (exact)."""
    return decode_table(kv_format)[np.asarray(codes, dtype=np.uint8)]


def encode_e4m3fn(values: np.ndarray) -> np.ndarray:
    """Round float values to e4m3fn codes, round-to-nearest-even.

    Inputs must already lie in [-448, 448] (the reference clamps first,
    ``smoke_cuda_paged_fp8_decode_op.py:16-18``); NaN maps to 0x7F.
    """
    x = np.asarray(values, dtype=np.float64)
    if np.any(np.abs(x[~np.isnan(x)]) > FP8_E4M3FN_MAX):
        raise ValueError("encode_e4m3fn expects values clamped to +-448")
    magnitude = np.abs(x)
    nan = np.isnan(magnitude)
    magnitude = np.where(nan, 0.0, magnitude)
    upper = np.searchsorted(_POSITIVE, magnitude, side="left")
    upper = np.clip(upper, 0, len(_POSITIVE) - 1)
    lower = np.clip(upper - 1, 0, len(_POSITIVE) - 1)
    d_up = _POSITIVE[upper] - magnitude
    d_lo = magnitude - _POSITIVE[lower]
    pick_upper = (d_up < d_lo) | ((d_up == d_lo) & (upper % 2 == 0))
    code = np.where(pick_upper, upper, lower).astype(np.uint8)
    code = np.where(np.signbit(x) & ~nan, code | 0x80, code)
    code = np.where(nan, 0x7F, code)
    return code.astype(np.uint8)


def quantize_fp8_e4m3(tensor: np.ndarray, floor: float = 1.0e-12) -> Tuple[np.ndarray, float]:
    """Per-tensor quantisation (``smoke_cuda_paged_fp8_decode_op.py:13-19``).

    Returns ``(codes, scale)`` with ``scale = max(amax / 448, floor)`` held as
    float32, and codes = RNE(clamp(x / scale, +-448)).
    """
    x = np.asarray(tensor, dtype=np.float32)
    scale = np.float32(max(float(np.abs(x).max()) / FP8_E4M3FN_MAX, floor))
    scaled = np.clip(x / scale, -FP8_E4M3FN_MAX, FP8_E4M3FN_MAX)
    return encode_e4m3fn(scaled), float(scale)


def quantize_fp8_e4m3_per_head(
    tensor: np.ndarray, head_axis: int = 2, floor: float = 1.0e-12
) -> Tuple[np.ndarray, np.ndarray]:
    """Per-KV-head variant: the per-tensor rule applied to each head slice."""
    x = np.asarray(tensor, dtype=np.float32)
    moved = np.moveaxis(x, head_axis, 0)
    amax = np.abs(moved.reshape(moved.shape[0], -1)).max(axis=1)
    scales = np.maximum(amax / FP8_E4M3FN_MAX, floor).astype(np.float32)
    shape = [1] * x.ndim
    shape[head_axis] = -1
    scaled = np.clip(x / scales.reshape(shape), -FP8_E4M3FN_MAX, FP8_E4M3FN_MAX)
    return encode_e4m3fn(scaled), scales


# --------------------------------------------------------------------------
# Paged gather + attention
# --------------------------------------------------------------------------
def _head_scales(scale: ScaleLike, num_kv_heads: int) -> np.ndarray:
    arr = np.asarray(scale, dtype=np.float32).reshape(-1)
    if arr.size == 1:
        return np.full(num_kv_heads, arr[0], dtype=np.float32)
    if arr.size != num_kv_heads:
        raise ValueError("per-head scale must have one entry per KV head")
    return arr


def gather_pages(cache: np.ndarray, table_row: np.ndarray, length: int) -> np.ndarray:
    """Logical tokens ``0..length-1`` of one sequence: ``cache[table[t // P], t % P]``
    for a cache of ``P``-token pages ``[pages, P, Hkv, D]`` (``P = cache.shape[1]``; the
    reference hook's page geometry, ``integrations/vllm/l20_paged_split_kv.py:156,182-200``)."""
    page = cache.shape[1]
    token = np.arange(length)
    physical = np.asarray(table_row)[token // page]
    return cache[physical, token % page]


def dequantize(codes: np.ndarray, scale: ScaleLike, head_axis: int = -2, kv_format: str = "e4m3fn") -> np.ndarray:
    """fp32 ``code * scale`` (one rounding), per tensor or per KV head."""
    values = fp8_to_f32(codes, kv_format)
    heads = values.shape[head_axis]
    scales = _head_scales(scale, heads)
    shape = [1] * values.ndim
    shape[head_axis] = heads
    return (values * scales.reshape(shape)).astype(np.float32)


def _tree_row(tree_mask: Optional[np.ndarray], b: int) -> Optional[np.ndarray]:
    if tree_mask is None:
        return None
    tm = np.asarray(tree_mask)
    return tm if tm.ndim == 1 else tm[b]


def tree_bits_from_mask(ancestor_mask: np.ndarray) -> np.ndarray:
    """Boolean ancestor matrix [..., S, S] (row i sees draft j) -> int64 bitmasks [..., S]."""
    m = np.asarray(ancestor_mask, dtype=bool)
    weights = (np.int64(1) << np.arange(m.shape[-1], dtype=np.int64))
    return (m.astype(np.int64) * weights).sum(-1)


def table_row(block_table: np.ndarray, b: int, page_indptr: Optional[np.ndarray] = None) -> np.ndarray:
    """Page list of sequence ``b``: row ``b`` of a ``[B, max_pages]`` block table, or
    ``page_indices[indptr[b]:indptr[b+1]]`` of a CSR page list
    (``l20_paged_decode.cu:205-208``: ``page_indptr[batch] + logical_page``)."""
    if page_indptr is None:
        return np.asarray(block_table[b])
    return np.asarray(block_table)[int(page_indptr[b]):int(page_indptr[b + 1])]


def tree_visibility(length: int, q_len: int, tree_bits: Optional[np.ndarray]) -> np.ndarray:
    """[q_len, L] visibility of one sequence's keys.  Without ``tree_bits`` row ``i``
    sees keys ``0 .. L - q_len + i`` (causal among the newest ``q_len``); with the
    per-row ancestor bitmasks ``tree_bits`` [q_len] row ``i`` sees the prefix
    ``0 .. L - q_len - 1`` and draft key ``L - q_len + j`` iff bit ``j`` of
    ``tree_bits[i]`` is set (``triton_tree_attention.py:1218-1240``: the cached
    prefix plus the ancestor mask over the suffix)."""
    token = np.arange(length)
    base = length - q_len
    if tree_bits is None:
        limit = base + np.arange(q_len)
        return token[None, :] <= limit[:, None]
    bits = np.asarray(tree_bits, dtype=np.int64).reshape(q_len, 1) & 0xFFFFFFFF
    draft = token[None, :] - base
    in_draft = draft >= 0
    bit = (bits >> np.clip(draft, 0, 31)) & 1
    return np.where(in_draft, bit == 1, True)


def _attend(query_rows: np.ndarray, keys: np.ndarray, values: np.ndarray, num_kv_heads: int,
            scale: float, q_len: int, acc_dtype, tree_bits: Optional[np.ndarray] = None
            ) -> Tuple[np.ndarray, np.ndarray]:
    """Softmax attention of one sequence's ``q_len`` query rows over its ``L`` keys with
    the visibility of ``tree_visibility``.  Returns (out [q, Hq, D], lse [q, Hq])."""
    length = keys.shape[0]
    _, num_q_heads, head_dim = query_rows.shape
    group = num_q_heads // num_kv_heads
    keys = keys.astype(acc_dtype)
    values = values.astype(acc_dtype)
    # [q, Hkv, G, D] x [L, Hkv, D] -> [q, Hkv, G, L]
    q = query_rows.reshape(q_len, num_kv_heads, group, head_dim)
    scores = np.einsum("ihgd,thd->ihgt", q.astype(acc_dtype), keys) * acc_dtype(scale)
    visible = tree_visibility(length, q_len, tree_bits)  # [q, L]
    scores = np.where(visible[:, None, None, :], scores, -np.inf)
    row_max = scores.max(axis=-1, keepdims=True)
    safe_max = np.where(np.isfinite(row_max), row_max, 0.0)
    weights = np.exp(scores - safe_max)
    denom = weights.sum(axis=-1, keepdims=True)
    probs = np.divide(weights, denom, out=np.zeros_like(weights), where=denom > 0)
    attended = np.einsum("ihgt,thd->ihgd", probs, values)
    with np.errstate(divide="ignore"):
        row_lse = (safe_max + np.log(denom))[..., 0]
    row_lse = np.where(denom[..., 0] > 0, row_lse, -np.inf)
    return attended.reshape(q_len, num_q_heads, head_dim), row_lse.reshape(q_len, num_q_heads)


def reference(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_table: np.ndarray,
    seq_lens: np.ndarray,
    k_scale: ScaleLike,
    v_scale: ScaleLike,
    *,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    round_kv_to: Optional[np.dtype] = None,
    acc_dtype: np.dtype = np.float32,
    rows: Optional[Sequence[int]] = None,
    page_indptr: Optional[np.ndarray] = None,
    tree_mask: Optional[np.ndarray] = None,
    kv_format: str = "e4m3fn",
) -> Tuple[np.ndarray, np.ndarray]:
    """Dequantise-then-attend (``smoke_cuda_paged_fp8_decode_op.py:22-41``).

    query       [B*q_len, Hq, D] float (bf16/fp16 values held as float32)
    key/value   [pages, P, Hkv, D] uint8 codes of ``kv_format`` (e4m3fn or e5m2), P-token pages
    block_table [B, max_pages] int (or the flat page list with ``page_indptr`` [B+1])
    seq_lens    [B] int;  k/v_scale float or [Hkv]
    Row ``b*q_len + i`` attends to keys ``0 .. L_b - q_len + i``.
    Returns ``(out [B*q_len, Hq, D] float32, lse [B*q_len, Hq] float32)``;
    rows with no visible key give zeros and ``lse = -inf``.
    ``rows`` restricts the work to the listed batch entries (others stay 0).
    ``tree_mask`` [B, q_len] (or [q_len], shared) int bitmasks replace the causal
    rule with an ancestor mask over the newest ``q_len`` keys.
    """
    query = np.asarray(query, dtype=np.float32)
    n_rows, num_q_heads, head_dim = query.shape
    batch = n_rows // q_len
    num_kv_heads = key_cache.shape[2]
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = np.zeros((n_rows, num_q_heads, head_dim), dtype=np.float32)
    lse = np.full((n_rows, num_q_heads), -np.inf, dtype=np.float32)
    for b in (range(batch) if rows is None else rows):
        length = int(seq_lens[b])
        if length <= 0:
            continue
        pages = table_row(block_table, b, page_indptr)
        keys = dequantize(gather_pages(key_cache, pages, length), k_scale, kv_format=kv_format)
        values = dequantize(gather_pages(value_cache, pages, length), v_scale, kv_format=kv_format)
        if round_kv_to is not None:
            keys = keys.astype(round_kv_to).astype(np.float32)
            values = values.astype(round_kv_to).astype(np.float32)
        o, l = _attend(query[b * q_len:(b + 1) * q_len], keys, values, num_kv_heads, scale, q_len, acc_dtype,
                       _tree_row(tree_mask, b))
        out[b * q_len:(b + 1) * q_len] = o
        lse[b * q_len:(b + 1) * q_len] = l
    return out, lse


def reference_dense_kv(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_table: np.ndarray,
    seq_lens: np.ndarray,
    *,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    rows: Optional[Sequence[int]] = None,
    page_indptr: Optional[np.ndarray] = None,
    tree_mask: Optional[np.ndarray] = None,
) -> Tuple[np.ndarray, np.ndarray]:
    """The fp16/bf16-KV siblings (``smoke_cuda_paged_decode_op.py:13-29``,
    ``l20_paged_decode.cu:156-289``): the same attention over caches whose values are
    used as stored (fp16/bf16 values held as float32), no scales, fp32 accumulation."""
    query = np.asarray(query, dtype=np.float32)
    n_rows, num_q_heads, head_dim = query.shape
    batch = n_rows // q_len
    num_kv_heads = key_cache.shape[2]
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = np.zeros((n_rows, num_q_heads, head_dim), dtype=np.float32)
    lse = np.full((n_rows, num_q_heads), -np.inf, dtype=np.float32)
    for b in (range(batch) if rows is None else rows):
        length = int(seq_lens[b])
        if length <= 0:
            continue
        pages = table_row(block_table, b, page_indptr)
        keys = np.asarray(gather_pages(key_cache, pages, length), dtype=np.float32)
        values = np.asarray(gather_pages(value_cache, pages, length), dtype=np.float32)
        o, l = _attend(query[b * q_len:(b + 1) * q_len], keys, values, num_kv_heads, scale, q_len, np.float32,
                       _tree_row(tree_mask, b))
        out[b * q_len:(b + 1) * q_len] = o
        lse[b * q_len:(b + 1) * q_len] = l
    return out, lse


def split_reference(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_table: np.ndarray,
    seq_lens: np.ndarray,
    k_scale: ScaleLike,
    v_scale: ScaleLike,
    split_size: int,
    *,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    kv_format: str = "e4m3fn",
) -> Tuple[np.ndarray, np.ndarray]:
    """Split-KV partials and LSE merge in float64 (``l20_paged_decode.cu:291-463``).

    Split ``s`` of sequence ``b`` covers tokens ``[s*S, min((s+1)*S, L_b))``.
    Each split yields ``(acc_s, m_s, l_s)``; the merge computes
    ``M = max m_s``, ``c_s = exp(m_s - M)``, ``out = sum c_s acc_s / sum c_s l_s``.
    """
    query = np.asarray(query, dtype=np.float64)
    n_rows, num_q_heads, head_dim = query.shape
    batch = n_rows // q_len
    num_kv_heads = key_cache.shape[2]
    group = num_q_heads // num_kv_heads
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = np.zeros((n_rows, num_q_heads, head_dim))
    lse = np.full((n_rows, num_q_heads), -np.inf)
    for b in range(batch):
        length = int(seq_lens[b])
        if length <= 0:
            continue
        keys = dequantize(gather_pages(key_cache, block_table[b], length), k_scale,
                          kv_format=kv_format).astype(np.float64)
        values = dequantize(gather_pages(value_cache, block_table[b], length), v_scale,
                            kv_format=kv_format).astype(np.float64)
        kv_of_head = np.arange(num_q_heads) // group
        for i in range(q_len):
            r = b * q_len + i
            limit = length - q_len + i
            partials = []
            for start in range(0, length, split_size):
                stop = min(start + split_size, length)
                tok = np.arange(start, stop)
                s = np.einsum("hd,thd->ht", query[r], keys[start:stop][:, kv_of_head]) * scale
                s = np.where(tok[None, :] <= limit, s, -np.inf)
                m = s.max(axis=1)
                safe = np.where(np.isfinite(m), m, 0.0)
                p = np.exp(s - safe[:, None])
                acc = np.einsum("ht,thd->hd", p, values[start:stop][:, kv_of_head])
                partials.append((acc, m, p.sum(axis=1)))
            m_all = np.stack([p[1] for p in partials])  # [n_s, Hq]
            big = m_all.max(axis=0)
            safe_big = np.where(np.isfinite(big), big, 0.0)
            corr = np.exp(m_all - safe_big)  # exp(-inf) = 0 for empty splits
            denom = sum(c * p[2] for c, p in zip(corr, partials))
            numer = sum(c[:, None] * p[0] for c, p in zip(corr, partials))
            ok = denom > 0
            out[r] = np.where(ok[:, None], numer / np.where(ok, denom, 1.0)[:, None], 0.0)
            with np.errstate(divide="ignore"):
                lse[r] = np.where(ok, safe_big + np.log(np.where(ok, denom, 1.0)), -np.inf)
    return out.astype(np.float32), lse.astype(np.float32)


def brute_force_fp64(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_table: np.ndarray,
    seq_lens: np.ndarray,
    k_scale: ScaleLike,
    v_scale: ScaleLike,
    *,
    softmax_scale: Optional[float] = None,
    q_len: int = 1,
    tree_mask: Optional[np.ndarray] = None,
    kv_format: str = "e4m3fn",
) -> Tuple[np.ndarray, np.ndarray]:
    """Scalar float64 loops, written independently of ``reference``; tiny inputs only."""
    n_rows, num_q_heads, head_dim = np.asarray(query).shape
    num_kv_heads = key_cache.shape[2]
    group = num_q_heads // num_kv_heads
    ks = _head_scales(k_scale, num_kv_heads)
    vs = _head_scales(v_scale, num_kv_heads)
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    decode = [float(v) for v in (e4m3fn_decode_table() if kv_format == "e4m3fn" else e5m2_decode_table())]
    out = np.zeros((n_rows, num_q_heads, head_dim))
    lse = np.full((n_rows, num_q_heads), -np.inf)
    page_tokens = key_cache.shape[1]
    for r in range(n_rows):
        b, i = divmod(r, q_len)
        length = int(seq_lens[b])
        last = length - q_len + i
        if tree_mask is None:
            keys = list(range(last + 1))
        else:  # prefix, then the draft keys whose bit is set in row i's ancestor word
            word = int(np.asarray(tree_mask).reshape(-1, q_len)[0 if np.asarray(tree_mask).ndim == 1 else b][i])
            keys = [t for t in range(length) if t < length - q_len or (word >> (t - (length - q_len))) & 1]
        for h in range(num_q_heads):
            kvh = h // group
            scores = []
            for t in keys:
                page = int(block_table[b][t // page_tokens])
                slot = t % page_tokens
                dot = 0.0
                for d in range(head_dim):
                    k = decode[int(key_cache[page, slot, kvh, d])] * float(ks[kvh])
                    dot += float(query[r, h, d]) * k
                scores.append(dot * scale)
            if not scores:
                continue
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = sum(weights)
            lse[r, h] = top + math.log(total)
            for t, w in zip(keys, weights):
                page = int(block_table[b][t // page_tokens])
                slot = t % page_tokens
                for d in range(head_dim):
                    v = decode[int(value_cache[page, slot, kvh, d])] * float(vs[kvh])
                    out[r, h, d] += w / total * v
    return out, lse
