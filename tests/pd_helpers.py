"""Helpers shared by the GPU parity tests, smoke() and bench.py's checks:
build seeded inputs, run the HIP op (torch dispatcher or C ABI), run the CPU
oracle on the same bytes, and compare to the stated tolerances.

Tolerances (bf16/fp16 output vs the fp32 dequantise-then-attend oracle):
max |diff| <= 1e-2 and per-(row, head) cosine >= 0.9999; natural-log LSE
|diff| <= 1e-4 * max(1, |lse|).  FP8 -> fp32 dequantisation is exact, so only
accumulation order (and the ~22-bit hi + lo split of the softmax probabilities
on the MFMA path) separates the two.
"""

from __future__ import annotations

import sys
from pathlib import Path
from typing import Optional, Sequence

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "single-gpu-inference-lab_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

OUT_ATOL = 1e-2
COS_MIN = 0.9999
LSE_RTOL = 1e-4


def quantize_e5m2(raw, per_head_axis=None):
    """OCP e5m2 codes of ``raw`` with the e4m3 quantiser's rule scaled to e5m2's
    largest finite value 57344: ``scale = max(amax / 57344, 1e-12)``."""
    xf = raw.float()
    if per_head_axis is None:
        scale = max(float(xf.abs().max()) / 57344.0, 1e-12)
        return (xf / scale).clamp(-57344.0, 57344.0).to(torch.float8_e5m2), scale
    moved = xf.movedim(per_head_axis, 0)
    scales = torch.clamp(moved.reshape(moved.shape[0], -1).abs().amax(dim=1) / 57344.0, min=1e-12)
    shape = [1] * xf.dim()
    shape[per_head_axis] = -1
    return (xf / scales.view(shape)).clamp(-57344.0, 57344.0).to(torch.float8_e5m2), scales


def kv_format(cache) -> str:
    """Oracle name of an fp8 cache's format."""
    return "e5m2" if cache.dtype == torch.float8_e5m2 else "e4m3fn"


def make_synthetic(batch, hq, hkv, d, lens, *, q_len=1, per_head=False, seed=0, device="cuda",
                   dtype=torch.bfloat16, pool_extra=7, max_pages=None, garbage_tail=False, fp8="e4m3fn",
                   page=16):
    """Seeded paged inputs of an arbitrary shape (generated on CPU, copied to ``device``).

    ``fp8`` picks the cache format: "e4m3fn" (the reference's quantiser) or "e5m2";
    ``page`` the tokens per page (caches [pages, page, Hkv, D])."""
    import l20_pd_workloads as wl

    g = torch.Generator().manual_seed(seed)
    lens = torch.as_tensor(lens, dtype=torch.int32)
    pages_per = (lens.to(torch.int64) + page - 1) // page
    pool = int(pages_per.sum()) + pool_extra
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    mp = max(1, int(pages_per.max())) if max_pages is None else max_pages
    table = torch.full((batch, mp), -7, dtype=torch.int32)  # unused entries are garbage
    off = 0
    for b in range(batch):
        n = int(pages_per[b])
        table[b, :n] = perm[off:off + n]
        off += n
    query = torch.randn(batch * q_len, hq, d, generator=g).to(dtype)
    caches = []
    for _ in range(2):
        raw = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16)
        if fp8 == "e5m2":
            codes, scale = quantize_e5m2(raw, per_head_axis=2 if per_head else None)
        else:
            codes, scale = wl.quantize_fp8_e4m3(raw, per_head_axis=2 if per_head else None)
        if garbage_tail:
            # bytes beyond each sequence's end in its last page: NaN codes
            u8 = codes.view(torch.uint8)
            for b in range(batch):
                L = int(lens[b])
                if L % page:
                    u8[int(table[b, L // page]), L % page:] = 0x7F
        caches.append((codes, scale))
    (kc, ks), (vc, vs) = caches
    return {
        "query": query.to(device), "key_cache": kc.to(device), "value_cache": vc.to(device),
        "block_table": table.to(device), "seq_lens": lens.to(device),
        "k_scale": ks if isinstance(ks, float) else ks.to(device),
        "v_scale": vs if isinstance(vs, float) else vs.to(device),
        "softmax_scale": d ** -0.5, "q_len": q_len, "max_seq_len": int(lens.max()) if len(lens) else 0,
    }


def _host_tree(inp):
    t = inp.get("tree_mask")
    return None if t is None else t.cpu().numpy().astype(np.int64)


def _scales(x):
    return (x, None) if isinstance(x, float) else (1.0, x)


def workspace(inp, split_size, partial_dtype=torch.float32, extra_splits=0):
    import math

    q = inp["query"]
    n_s = max(1, math.ceil(inp["max_seq_len"] / split_size)) + extra_splits
    rows, hq, d = q.shape
    return (torch.empty(rows, hq, n_s, d, dtype=partial_dtype, device=q.device),
            torch.empty(rows, hq, n_s, dtype=torch.float32, device=q.device),
            torch.empty(rows, hq, n_s, dtype=torch.float32, device=q.device))


def run_op(inp, split_size, *, via="torch", partial_dtype=torch.float32, with_lse=True, key_cache=None,
           value_cache=None, output=None):
    """Run the HIP op on ``inp``; returns ``(out, lse)`` (device tensors)."""
    import l20_paged_decode  # noqa: F401
    import l20_pd_cabi as cabi

    q = inp["query"]
    kc = inp["key_cache"] if key_cache is None else key_cache
    vc = inp["value_cache"] if value_cache is None else value_cache
    po, pm, ps = workspace(inp, split_size, partial_dtype)
    out = torch.empty_like(q) if output is None else output
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device) if with_lse else None
    ks, ksph = _scales(inp["k_scale"])
    vs, vsph = _scales(inp["v_scale"])
    if via == "torch":
        torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
            q, kc, vc, inp["block_table"], inp["seq_lens"], po, pm, ps, out, ks, vs,
            inp["max_seq_len"], split_size, inp["softmax_scale"], ksph, vsph, inp["q_len"], lse,
            inp.get("tree_mask"))
    else:
        args = cabi.args_from_tensors(
            q, kc, vc, inp["block_table"], inp["seq_lens"], po, pm, ps, out, ks, vs, inp["max_seq_len"],
            split_size, softmax_scale=inp["softmax_scale"], k_scale_per_head=ksph, v_scale_per_head=vsph,
            q_len=inp["q_len"], lse=lse, tree_mask=inp.get("tree_mask"))
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, lse


def run_oracle(inp, rows: Optional[Sequence[int]] = None):
    """The CPU oracle on the same bytes; returns numpy ``(out, lse)``."""
    from oracle import paged_fp8_decode_ref as ref

    def host_scale(s):
        return s if isinstance(s, float) else s.float().cpu().numpy()

    return ref.reference(
        inp["query"].float().cpu().numpy(),
        inp["key_cache"].view(torch.uint8).cpu().numpy(),
        inp["value_cache"].view(torch.uint8).cpu().numpy(),
        inp["block_table"].cpu().numpy(),
        inp["seq_lens"].cpu().numpy(),
        host_scale(inp["k_scale"]), host_scale(inp["v_scale"]),
        softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], rows=rows, tree_mask=_host_tree(inp),
        kv_format=kv_format(inp["key_cache"]))


def compare(out, lse, exp_out, exp_lse, rows: Optional[np.ndarray] = None, check_lse=True):
    """Assert the tolerances; returns a dict of the observed errors."""
    got = out.float().cpu().numpy()
    got_lse = lse.cpu().numpy() if lse is not None else None
    if rows is not None:
        got, exp_out = got[rows], exp_out[rows]
        if got_lse is not None:
            got_lse, exp_lse = got_lse[rows], exp_lse[rows]
    assert np.all(np.isfinite(got)), "non-finite output"
    diff = np.abs(got - exp_out)
    max_abs = float(diff.max()) if diff.size else 0.0
    num = (got * exp_out).sum(-1)
    den = np.linalg.norm(got, axis=-1) * np.linalg.norm(exp_out, axis=-1)
    nz = den > 0
    cos = np.where(nz, num / np.where(nz, den, 1.0), 1.0)
    # rows whose expected output is exactly zero must be zero too
    assert np.all(np.abs(got[~nz]) <= OUT_ATOL)
    min_cos = float(cos.min()) if cos.size else 1.0
    res = {"max_abs": max_abs, "min_cos": min_cos}
    assert max_abs <= OUT_ATOL, res
    assert min_cos >= COS_MIN, res
    if check_lse and got_lse is not None:
        both_inf = np.isneginf(got_lse) & np.isneginf(exp_lse)
        assert np.array_equal(np.isneginf(got_lse), np.isneginf(exp_lse)), "LSE -inf pattern differs"
        fin = ~both_inf
        err = np.abs(got_lse[fin] - exp_lse[fin]) / np.maximum(1.0, np.abs(exp_lse[fin]))
        res["lse_rel"] = float(err.max()) if err.size else 0.0
        assert res["lse_rel"] <= LSE_RTOL, res
    return res


# ------------------------------------------------------------ 16-bit caches, CSR page lists
def make_synthetic16(batch, hq, hkv, d, lens, *, dtype=torch.float16, q_len=1, seed=0, device="cuda",
                     pool_extra=7, garbage_tail=False, csr_pad=0, page=16):
    """Seeded inputs for the fp16/bf16-KV siblings: query and caches of ``dtype``, a
    block table and the same pages as a CSR list (``csr_pad`` garbage entries after
    each row, so that offsets and not row lengths are exercised)."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.as_tensor(lens, dtype=torch.int32)
    pages_per = (lens.to(torch.int64) + page - 1) // page
    pool = int(pages_per.sum()) + pool_extra
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    mp = max(1, int(pages_per.max()))
    table = torch.full((batch, mp), -7, dtype=torch.int32)
    indices, indptr = [], [0]
    off = 0
    for b in range(batch):
        n = int(pages_per[b])
        table[b, :n] = perm[off:off + n]
        indices.append(perm[off:off + n])
        if csr_pad:
            indices.append(torch.full((csr_pad,), 10**6, dtype=torch.int32))
        indptr.append(indptr[-1] + n + csr_pad)
        off += n
    query = torch.randn(batch * q_len, hq, d, generator=g).to(dtype)
    kc = torch.randn(pool, page, hkv, d, generator=g).to(dtype)
    vc = torch.randn(pool, page, hkv, d, generator=g).to(dtype)
    if garbage_tail:
        for c in (kc, vc):
            for b in range(batch):
                L = int(lens[b])
                if L % page:
                    c[int(table[b, L // page]), L % page:] = float("nan")
    return {
        "query": query.to(device), "key_cache": kc.to(device), "value_cache": vc.to(device),
        "block_table": table.to(device), "seq_lens": lens.to(device),
        "page_indices": (torch.cat(indices) if indices else torch.zeros(0, dtype=torch.int32)).to(device),
        "page_indptr": torch.tensor(indptr, dtype=torch.int32).to(device),
        "softmax_scale": None, "q_len": q_len, "max_seq_len": int(lens.max()) if len(lens) else 0,
    }


def run_op16(inp, split_size, *, via="torch", csr=False, partial_dtype=torch.float32, with_lse=True):
    """Run the 16-bit-cache sibling (block table or CSR); returns ``(out, lse)``."""
    import l20_paged_decode  # noqa: F401
    import l20_pd_cabi as cabi

    q = inp["query"]
    po, pm, ps = workspace(inp, split_size, partial_dtype)
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device) if with_lse else None
    if via == "torch":
        if csr:
            torch.ops.l20_stack.paged_decode_split_indices_out(
                q, inp["key_cache"], inp["value_cache"], inp["page_indptr"], inp["page_indices"], inp["seq_lens"],
                po, pm, ps, out, inp["max_seq_len"], split_size, inp["softmax_scale"], inp["q_len"], lse,
                inp.get("tree_mask"))
        else:
            torch.ops.l20_stack.paged_decode_split_out(
                q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"], po, pm, ps, out,
                inp["max_seq_len"], split_size, inp["softmax_scale"], inp["q_len"], lse, inp.get("tree_mask"))
    else:
        table = inp["page_indices"] if csr else inp["block_table"]
        args = cabi.args_from_tensors(
            q, inp["key_cache"], inp["value_cache"], table, inp["seq_lens"], po, pm, ps, out, 1.0, 1.0,
            inp["max_seq_len"], split_size, softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], lse=lse,
            page_indptr=inp["page_indptr"] if csr else None, tree_mask=inp.get("tree_mask"))
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, lse


def run_oracle16(inp, rows: Optional[Sequence[int]] = None, csr=False):
    """The CPU oracle for 16-bit caches on the same values; numpy ``(out, lse)``."""
    from oracle import paged_fp8_decode_ref as ref

    table = inp["page_indices"] if csr else inp["block_table"]
    return ref.reference_dense_kv(
        inp["query"].float().cpu().numpy(), inp["key_cache"].float().cpu().numpy(),
        inp["value_cache"].float().cpu().numpy(), table.cpu().numpy(), inp["seq_lens"].cpu().numpy(),
        softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], rows=rows,
        page_indptr=inp["page_indptr"].cpu().numpy() if csr else None, tree_mask=_host_tree(inp))


# ------------------------------------------------------------ tree attention oracles
def dense_tree_oracle(query, prefix_k, prefix_v, suffix_k, suffix_v, mask, scale):
    """fp64 attention over concat(prefix, suffix) keys: every row sees the prefix,
    row i sees draft j iff mask[i, j] (any draft count, unlike the 32-bit words)."""
    b, s, hq, d = query.shape
    hkv = prefix_k.shape[2]
    g = hq // hkv
    p = prefix_k.shape[1]
    visible = np.concatenate([np.ones((s, p), dtype=bool), mask], 1)  # [S, P+S]
    out = np.zeros((b, s, hq, d))
    for i in range(b):
        keys = np.concatenate([prefix_k[i], suffix_k[i]], 0).astype(np.float64)
        vals = np.concatenate([prefix_v[i], suffix_v[i]], 0).astype(np.float64)
        q = query[i].astype(np.float64).reshape(s, hkv, g, d)
        sc = np.einsum("ihgd,thd->ihgt", q, keys) * scale
        sc = np.where(visible[:, None, None, :], sc, -np.inf)
        w = np.exp(sc - sc.max(-1, keepdims=True))
        w /= w.sum(-1, keepdims=True)
        out[i] = np.einsum("ihgt,thd->ihgd", w, vals).reshape(s, hq, d)
    return out


def paged_tree_oracle(query, prefix_k, prefix_v, suffix_k, suffix_v, mask, scale, page=16):
    """The pinned oracle (``oracle.paged_fp8_decode_ref.reference_dense_kv`` with tree
    words) over the prefix keys followed by the draft keys, laid out as ``page``-token
    pages of one float32 cache: ``(out [B, S, Hq, D], lse [B, S, Hq])``.  With an
    all-False ``mask`` the rows see the prefix alone (the prefix pass's LSE)."""
    from oracle import paged_fp8_decode_ref as ref

    b, s, hq, d = query.shape
    hkv = prefix_k.shape[2]
    cached = prefix_k.shape[1]
    length = cached + s
    per = max(1, -(-length // page))
    table = np.arange(b * per, dtype=np.int32).reshape(b, per)[:, ::-1].copy()  # pages out of order
    kc = np.zeros((b * per, page, hkv, d), np.float32)
    vc = np.zeros_like(kc)
    for i in range(b):
        keys = np.concatenate([prefix_k[i], suffix_k[i]], 0)
        vals = np.concatenate([prefix_v[i], suffix_v[i]], 0)
        for t in range(length):
            kc[table[i, t // page], t % page] = keys[t]
            vc[table[i, t // page], t % page] = vals[t]
    m = np.asarray(mask, dtype=bool)
    words = (m.astype(np.int64) << np.arange(s, dtype=np.int64)).sum(1)  # row i: bit j iff mask[i, j]
    out, lse = ref.reference_dense_kv(query.reshape(b * s, hq, d), kc, vc, table, np.full(b, length), q_len=s,
                                      softmax_scale=scale, tree_mask=words)
    return out.reshape(b, s, hq, d), lse.reshape(b, s, hq)
