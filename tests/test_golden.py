"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle, re-run on each fixture's stored inputs, reproduces the
stored outputs exactly (a regression pin on oracle/).  GPU: the HIP op on the
same inputs matches them to the usual tolerances (fp8 / 16-bit decode, verify,
tree words, CSR page lists) or bit for bit (the KV producer).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

import pd_helpers as H
from oracle import kv_write_ref as kref
from oracle import paged_fp8_decode_ref as ref

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem for p in GOLDEN.glob("*.npz"))
# GPU cases: each attention fixture at two split sizes; the KV producer takes no split.
GPU_CASES = [(name, split) for name in CASES
             for split in ((0,) if name.startswith("kv_write") else (64, 1024))]


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))


def bf16(bits):
    return torch.from_numpy(bits).view(torch.bfloat16)


def _oracle(f):
    kind = str(f["kind"])
    if kind == "fp8":
        q = bf16(f["query_bf16"]).float().numpy()
        ks = f["k_scale"] if f["k_scale"].ndim else float(f["k_scale"])
        vs = f["v_scale"] if f["v_scale"].ndim else float(f["v_scale"])
        tree = f["tree_mask"].astype(np.int64) if f["tree_mask"].size else None
        return ref.reference(q, f["key_codes"], f["value_codes"], f["block_table"], f["seq_lens"], ks, vs,
                             softmax_scale=float(f["softmax_scale"]), q_len=int(f["q_len"]), tree_mask=tree)
    if kind == "kv16":
        dt = torch.bfloat16 if str(f["dtype"]) == "bfloat16" else torch.float16
        as_f = lambda b: torch.from_numpy(b).view(dt).float().numpy()  # noqa: E731
        return ref.reference_dense_kv(as_f(f["query_bits"]), as_f(f["key_bits"]), as_f(f["value_bits"]),
                                      f["page_indices"], f["seq_lens"], softmax_scale=None, q_len=int(f["q_len"]),
                                      page_indptr=f["page_indptr"])
    kc0 = np.zeros((int(f["pages"]), 16) + f["key_bf16"].shape[1:], dtype=np.uint8)
    return kref.rope_and_cache(bf16(f["query_bf16"]).float().numpy(), bf16(f["key_bf16"]).float().numpy(),
                               bf16(f["value_bf16"]).float().numpy(), f["positions"],
                               bf16(f["cos_sin_bf16"]).float().numpy(), bool(f["is_neox"]), kc0, kc0.copy(),
                               f["slots"], dtype="bf16", cache_fp8=True, k_scale=f["k_scale"], v_scale=f["v_scale"])


def test_golden_fixtures_present():
    assert len(CASES) >= 6, CASES


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    f = load(name)
    got = _oracle(f)
    if str(f["kind"]) == "kv_write":
        for g, key in zip(got, ("expected_query", "expected_key", "expected_key_cache", "expected_value_cache")):
            assert np.array_equal(g, f[key]), key
    else:
        out, lse = got
        assert np.array_equal(out.astype(np.float32), f["expected_out"])
        assert np.array_equal(lse.astype(np.float32), f["expected_lse"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,split", GPU_CASES)
def test_hip_op_matches_golden(name, split):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    import l20_paged_decode  # noqa: F401
    import l20_rope_kv

    f = load(name)
    kind = str(f["kind"])
    dev = "cuda"
    if kind == "kv_write":
        q, k = bf16(f["query_bf16"]).to(dev), bf16(f["key_bf16"]).to(dev)
        v = bf16(f["value_bf16"]).to(dev)
        kc = torch.zeros((int(f["pages"]), 16) + tuple(f["key_bf16"].shape[1:]), dtype=torch.float8_e4m3fn,
                         device=dev)
        vc = torch.zeros_like(kc)
        l20_rope_kv.l20_rope_and_cache(q, k, v, torch.from_numpy(f["positions"]).to(dev),
                                       bf16(f["cos_sin_bf16"]).to(dev), bool(f["is_neox"]), kc, vc,
                                       torch.from_numpy(f["slots"]).to(dev),
                                       k_scale_per_head=torch.from_numpy(f["k_scale"]).to(dev),
                                       v_scale_per_head=torch.from_numpy(f["v_scale"]).to(dev))
        torch.cuda.synchronize()
        assert np.array_equal(q.float().cpu().numpy(), f["expected_query"])
        assert np.array_equal(k.float().cpu().numpy(), f["expected_key"])
        assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), f["expected_key_cache"])
        assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), f["expected_value_cache"])
        return
    q_len = int(f["q_len"])
    lens = f["seq_lens"]
    common = {"seq_lens": torch.from_numpy(lens).to(dev), "q_len": q_len,
              "max_seq_len": int(lens.max()) if lens.size else 0}
    if kind == "fp8":
        inp = dict(common, query=bf16(f["query_bf16"]).to(dev),
                   key_cache=torch.from_numpy(f["key_codes"]).view(torch.float8_e4m3fn).to(dev),
                   value_cache=torch.from_numpy(f["value_codes"]).view(torch.float8_e4m3fn).to(dev),
                   block_table=torch.from_numpy(f["block_table"]).to(dev),
                   k_scale=float(f["k_scale"]) if not f["k_scale"].ndim else torch.from_numpy(f["k_scale"]).to(dev),
                   v_scale=float(f["v_scale"]) if not f["v_scale"].ndim else torch.from_numpy(f["v_scale"]).to(dev),
                   softmax_scale=float(f["softmax_scale"]))
        if f["tree_mask"].size:
            inp["tree_mask"] = torch.from_numpy(f["tree_mask"]).to(dev)
        out, lse = H.run_op(inp, split)
    else:
        dt = torch.bfloat16 if str(f["dtype"]) == "bfloat16" else torch.float16
        inp = dict(common, query=torch.from_numpy(f["query_bits"]).view(dt).to(dev),
                   key_cache=torch.from_numpy(f["key_bits"]).view(dt).to(dev),
                   value_cache=torch.from_numpy(f["value_bits"]).view(dt).to(dev),
                   block_table=torch.from_numpy(f["block_table"]).to(dev),
                   page_indices=torch.from_numpy(f["page_indices"]).to(dev),
                   page_indptr=torch.from_numpy(f["page_indptr"]).to(dev), softmax_scale=None)
        out, lse = H.run_op16(inp, split, csr=True)
    H.compare(out, lse, f["expected_out"], f["expected_lse"])
