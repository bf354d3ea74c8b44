#!/usr/bin/env python3
"""Writes the golden fixtures in this directory: small seeded inputs of the
paged decode op (fp8 and 16-bit caches, decode / verify / tree) and of the KV
producer, each with the CPU oracle's expected outputs.

The reference repository holds no numeric vectors for this path, so the
expected outputs come from this build's oracle (oracle/), itself pinned by
closed forms, invariants and brute force (tests/test_oracle.py).  The
fixtures freeze those outputs: tests/test_golden.py re-runs the oracle on
the stored inputs (CPU) and runs the HIP op on them (GPU).

    python tests/golden/make_golden.py      # rewrites the .npz files
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (str(ROOT / "single-gpu-inference-lab_amd"), str(ROOT), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import pd_helpers as H  # noqa: E402
from oracle import kv_write_ref as kref  # noqa: E402
from oracle import paged_fp8_decode_ref as ref  # noqa: E402

# name: (batch, hq, hkv, d, lens, q_len, per_head, seed, tree)
FP8_CASES = {
    "fp8_decode_d64": (4, 14, 2, 64, [64, 100, 33, 17], 1, False, 29, False),
    "fp8_verify_q4_per_head": (3, 8, 2, 128, [70, 4, 130], 4, True, 31, False),
    "fp8_tree_q4": (2, 8, 2, 128, [150, 40], 4, False, 37, True),
}
# name: (batch, hq, hkv, d, lens, q_len, dtype, seed)
KV16_CASES = {
    "bf16_decode_csr": (3, 16, 2, 64, [33, 90, 16], 1, torch.bfloat16, 41),
    "fp16_verify_q2": (2, 8, 2, 64, [65, 100], 2, torch.float16, 43),
}
TREE_WORDS = np.array([[1, 3, 5, 11], [1, 2, 6, 12]], dtype=np.int32)  # two ancestor trees of 4 drafts


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy()


def fp8_case(name, batch, hq, hkv, d, lens, q_len, per_head, seed, tree):
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, seed=seed, device="cpu",
                           garbage_tail=True, pool_extra=1)
    if tree:
        inp["tree_mask"] = torch.from_numpy(TREE_WORDS[:batch])
    ks = inp["k_scale"] if isinstance(inp["k_scale"], float) else inp["k_scale"].numpy()
    vs = inp["v_scale"] if isinstance(inp["v_scale"], float) else inp["v_scale"].numpy()
    out, lse = ref.reference(inp["query"].float().numpy(), inp["key_cache"].view(torch.uint8).numpy(),
                             inp["value_cache"].view(torch.uint8).numpy(), inp["block_table"].numpy(),
                             inp["seq_lens"].numpy(), ks, vs, softmax_scale=inp["softmax_scale"], q_len=q_len,
                             tree_mask=TREE_WORDS[:batch].astype(np.int64) if tree else None)
    np.savez_compressed(HERE / f"{name}.npz", kind="fp8", query_bf16=bits16(inp["query"]),
                        key_codes=inp["key_cache"].view(torch.uint8).numpy(),
                        value_codes=inp["value_cache"].view(torch.uint8).numpy(),
                        block_table=inp["block_table"].numpy(), seq_lens=inp["seq_lens"].numpy(),
                        k_scale=np.asarray(ks, dtype=np.float32), v_scale=np.asarray(vs, dtype=np.float32),
                        softmax_scale=np.float32(inp["softmax_scale"]), q_len=q_len,
                        tree_mask=TREE_WORDS[:batch] if tree else np.zeros((0,), np.int32),
                        expected_out=out.astype(np.float32), expected_lse=lse.astype(np.float32))


def kv16_case(name, batch, hq, hkv, d, lens, q_len, dtype, seed):
    inp = H.make_synthetic16(batch, hq, hkv, d, lens, dtype=dtype, q_len=q_len, seed=seed, device="cpu",
                             garbage_tail=True, csr_pad=1, pool_extra=1)
    out, lse = ref.reference_dense_kv(inp["query"].float().numpy(), inp["key_cache"].float().numpy(),
                                      inp["value_cache"].float().numpy(), inp["page_indices"].numpy(),
                                      inp["seq_lens"].numpy(), softmax_scale=None, q_len=q_len,
                                      page_indptr=inp["page_indptr"].numpy())
    np.savez_compressed(HERE / f"{name}.npz", kind="kv16", dtype=str(dtype).split(".")[-1],
                        query_bits=bits16(inp["query"]), key_bits=bits16(inp["key_cache"]),
                        value_bits=bits16(inp["value_cache"]), block_table=inp["block_table"].numpy(),
                        page_indices=inp["page_indices"].numpy(), page_indptr=inp["page_indptr"].numpy(),
                        seq_lens=inp["seq_lens"].numpy(), q_len=q_len,
                        expected_out=out.astype(np.float32), expected_lse=lse.astype(np.float32))


def kv_write_case(name="kv_write_fp8_neox", tokens=37, hq=4, hkv=2, d=64, is_neox=True, seed=47):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(tokens, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(tokens, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(tokens, hkv, d, generator=g).to(torch.bfloat16)
    positions = torch.randint(0, 256, (tokens,), generator=g).to(torch.int64)
    theta = torch.rand(256, d // 2, generator=g, dtype=torch.float64) * 6.2831853
    cos_sin = torch.cat([theta.cos(), theta.sin()], -1).to(torch.bfloat16)
    pages = (tokens + 15) // 16 + 2
    slots = torch.randperm(pages * 16, generator=g)[:tokens].to(torch.int64)
    slots[5] = -1  # a padding token: skipped
    kc0 = np.zeros((pages, 16, hkv, d), dtype=np.uint8)
    ks = np.array([0.011, 0.009], dtype=np.float32)
    vs = np.array([0.008, 0.012], dtype=np.float32)
    q_out, k_out, kc, vc = kref.rope_and_cache(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                               positions.numpy(), cos_sin.float().numpy(), is_neox, kc0,
                                               kc0.copy(), slots.numpy(), dtype="bf16", cache_fp8=True,
                                               k_scale=ks, v_scale=vs)
    np.savez_compressed(HERE / f"{name}.npz", kind="kv_write", query_bf16=bits16(q), key_bf16=bits16(k),
                        value_bf16=bits16(v), positions=positions.numpy(), cos_sin_bf16=bits16(cos_sin),
                        slots=slots.numpy(), is_neox=is_neox, pages=pages, k_scale=ks, v_scale=vs,
                        expected_query=q_out.astype(np.float32), expected_key=k_out.astype(np.float32),
                        expected_key_cache=kc, expected_value_cache=vc)


def main():
    for name, c in FP8_CASES.items():
        fp8_case(name, *c)
    for name, c in KV16_CASES.items():
        kv16_case(name, *c)
    kv_write_case()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
