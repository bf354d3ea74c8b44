"""Split mode of the single-launch kernel (GPU): one 8-wave workgroup per
(split, sequence, KV head), wave w streaming the w-th eighth of the split,
the waves' online-softmax states folded in LDS and the split's partial
(o / l, m, l) written into the workspace for the merge kernel; a sequence of
one split writes its output rows directly.

* Forced with L20_PD_FUSED_SPLIT=1 on the shapes the mode accepts (fp8 e4m3 /
  e5m2 and fp16 / bf16 caches, block tables and CSR page lists, head_dim
  64 / 128, draft rows and ancestor trees over one and two query tiles, empty
  and ragged rows, pages of 16 / 32 / 64 tokens, per-head scales, splits of
  256, 512 and 1024 tokens: 1, 2 and 4 fp8 blocks per wave), over fp32, fp16
  and bf16 workspaces: output and LSE against the oracle, through the C ABI.
* The library's own choice at config 2 (its default split of 512 takes the
  mode) at full size, and at 256- and 1024-token splits (8 x 2048 and 8 x 8192
  tokens, 4 KV heads), against the oracle.
* Graph capture: replays bitwise equal to the eager call; prior workspace
  contents (NaN) change nothing.
"""

import zlib

import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu

PDT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}

CASES = [
    # name, batch, hq, hkv, d, lens, q_len, per_head, fp8, page, split, pdt
    ("ragged_d128", 5, 28, 4, 128, [1, 15, 1025, 2048, 600], 1, True, "e4m3fn", 16, 512, "fp16"),
    ("ragged_fp32_ws", 4, 28, 4, 128, [3000, 17, 512, 513], 1, False, "e4m3fn", 16, 512, "fp32"),
    ("bf16_ws", 3, 16, 2, 128, [2000, 1, 700], 1, False, "e4m3fn", 16, 512, "bf16"),
    ("split256_1blk", 3, 16, 2, 128, [1500, 257, 31], 1, False, "e4m3fn", 16, 256, "fp32"),
    ("split1024_4blk", 2, 32, 8, 128, [5000, 1100], 1, True, "e4m3fn", 16, 1024, "fp16"),
    ("d64", 4, 14, 2, 64, [1500, 64, 0, 900], 1, False, "e4m3fn", 16, 512, "fp32"),
    ("empty_rows", 3, 8, 2, 128, [0, 1200, 0], 1, False, "e4m3fn", 16, 512, "fp32"),
    ("mha_g1", 2, 4, 4, 128, [1800, 90], 1, False, "e4m3fn", 16, 512, "fp16"),
    ("group16", 2, 32, 2, 128, [1290, 700], 1, False, "e4m3fn", 16, 512, "fp32"),
    ("e5m2", 4, 16, 2, 128, [1, 1333, 2048, 64], 1, True, "e5m2", 16, 512, "fp16"),
    ("pages_32", 4, 16, 2, 128, [1, 1000, 2049, 64], 1, False, "e4m3fn", 32, 512, "fp32"),
    ("pages_64", 3, 28, 4, 128, [900, 31, 2500], 1, True, "e4m3fn", 64, 512, "fp16"),
    ("verify_q4_g4", 3, 8, 2, 128, [1070, 4, 1513], 4, False, "e4m3fn", 16, 512, "fp32"),
    ("verify_2tiles", 4, 64, 8, 128, [2048, 17, 1300, 4], 4, False, "e4m3fn", 16, 512, "fp16"),
]


def _run(inp, split, pdt, table=None, indptr=None, kv_scales=None):
    """The C ABI with a NaN-filled workspace; returns (out, lse, path)."""
    import l20_pd_cabi as cabi

    po, pm, ps = H.workspace(inp, split, pdt)
    for t in (po, pm, ps):
        t.fill_(float("nan"))
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    if kv_scales is None:
        ks, ksph = H._scales(inp["k_scale"])
        vs, vsph = H._scales(inp["v_scale"])
    else:
        (ks, ksph), (vs, vsph) = kv_scales
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"],
                                  inp["block_table"] if table is None else table, inp["seq_lens"],
                                  po, pm, ps, out, ks, vs, inp["max_seq_len"], split,
                                  softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], lse=lse,
                                  k_scale_per_head=ksph, v_scale_per_head=vsph, tree_mask=inp.get("tree_mask"),
                                  page_indptr=indptr)
    path = cabi.launch_path(args)
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, lse, path


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_split_mode_matches_oracle(case, monkeypatch):
    name, batch, hq, hkv, d, lens, q_len, per_head, fp8, page, split, pdt = case
    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, fp8=fp8, page=page,
                           seed=zlib.crc32(name.encode()) % 1000, garbage_tail=True)
    out, lse, path = _run(inp, split, PDT[pdt])
    assert path == 2
    H.compare(out, lse, *H.run_oracle(inp))


@pytest.mark.parametrize("tree_case", [("tree_1tile", 3, 8, 2, [1700, 37, 1500]),
                                       ("tree_2tiles", 2, 16, 2, [2000, 1333])],
                         ids=lambda c: c[0])
def test_split_mode_tree_masks(tree_case, monkeypatch):
    """Random ancestor trees over the newest q_len keys (one and two query
    tiles), against the oracle's masked attention."""
    import numpy as np
    from test_gpu_tree_verify import random_tree, words

    name, batch, hq, hkv, lens = tree_case
    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    q_len = 4
    inp = H.make_synthetic(batch, hq, hkv, 128, lens, q_len=q_len, seed=zlib.crc32(name.encode()) % 1000,
                           garbage_tail=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    inp["tree_mask"] = words(np.stack([random_tree(q_len, rng) for _ in range(batch)])).cuda()
    out, lse, path = _run(inp, 512, torch.float32)
    assert path == 2
    H.compare(out, lse, *H.run_oracle(inp))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("csr", [False, True], ids=["table", "csr"])
def test_split_mode_16bit_caches(dtype, csr, monkeypatch):
    """16-bit caches (16-token blocks: 4 per wave at 512-token splits), block
    tables and CSR page lists, against the oracle."""
    import l20_pd_cabi as cabi

    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    inp = H.make_synthetic16(3, 16, 2, 128, [1500, 33, 2048], dtype=dtype, csr_pad=2, seed=11, garbage_tail=True)
    exp = H.run_oracle16(inp, csr=csr)
    po, pm, ps = H.workspace(inp, 512, torch.float32)
    for t in (po, pm, ps):
        t.fill_(float("nan"))
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    table = inp["page_indices"] if csr else inp["block_table"]
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], table, inp["seq_lens"], po, pm, ps, out,
                                  1.0, 1.0, inp["max_seq_len"], 512, softmax_scale=inp["softmax_scale"],
                                  lse=lse, page_indptr=inp["page_indptr"] if csr else None)
    assert cabi.launch_path(args) == 2
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    H.compare(out, lse, *exp)


def test_library_takes_the_split_mode_at_config_2(monkeypatch):
    """Config 2 (32 x 2048 tokens, 2 KV heads): the library's default split is
    512 and its partial stage the split mode; full size against the oracle,
    through the C ABI and the torch op."""
    import l20_pd_cabi as cabi
    import l20_pd_workloads as wl

    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    monkeypatch.delenv("L20_PD_FUSED_SPLIT", raising=False)
    cfg = wl.CONFIGS["c2_qwen2.5_coder_3b"]
    inp = wl.make_inputs(cfg, device="cuda")
    inp["query"] = inp["query"].contiguous()
    split = int(cabi.load().l20_pd_default_split_size(cfg.batch, cfg.num_kv_heads, inp["max_seq_len"], 0))
    assert split == 512
    exp = H.run_oracle(inp)
    out, lse, path = _run(inp, split, torch.float16,
                          kv_scales=(H._scales(inp["k_scale"]), H._scales(inp["v_scale"])))
    assert path == 2
    H.compare(out, lse, *exp)
    H.compare(*H.run_op(inp, split, partial_dtype=torch.float16), *exp)


def test_split_mode_graph_replays_and_prior_contents(monkeypatch):
    """Captured in a HIP graph and replayed three times with eager calls in
    between, every replay is bitwise equal to the eager call; so is a call
    over a workspace, output and LSE prefilled with NaN."""
    import l20_pd_cabi as cabi

    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    inp = H.make_synthetic(6, 28, 4, 128, [3000, 1, 1517, 64, 0, 2333], seed=12)
    split = 512
    po, pm, ps = H.workspace(inp, split, torch.float16)
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                  po, pm, ps, out, inp["k_scale"], inp["v_scale"], inp["max_seq_len"], split,
                                  softmax_scale=inp["softmax_scale"], lse=lse)
    assert cabi.launch_path(args) == 2
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = (out.clone(), lse.clone())
    H.compare(out, lse, *H.run_oracle(inp))
    for t in (po, pm, ps, out, lse):
        t.fill_(float("nan"))
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out, eager[0]) and torch.equal(lse, eager[1])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        cabi.split_out(args, side.cuda_stream)  # warm-up outside the capture
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            cabi.split_out(args, side.cuda_stream)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        lse.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]) and torch.equal(lse, eager[1])
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]) and torch.equal(lse, eager[1])


def test_library_takes_the_split_mode_at_1024_token_splits(monkeypatch):
    """8 x 8192 tokens, 28 query / 4 KV heads: 512 triples at 512-token splits,
    256 at 1024, so the library's split is 1024 and the partial stage the split
    mode (four fp8 blocks per wave); against the oracle."""
    import l20_pd_cabi as cabi

    monkeypatch.delenv("L20_PD_FUSED_SPLIT", raising=False)
    inp = H.make_synthetic(8, 28, 4, 128, [8192, 8000, 7001, 8192, 6500, 8192, 7777, 8100], seed=23)
    split = int(cabi.load().l20_pd_default_split_size(8, 4, inp["max_seq_len"], 0))
    assert split == 1024
    out, lse, path = _run(inp, split, torch.float16)
    assert path == 2
    H.compare(out, lse, *H.run_oracle(inp))


def test_noalloc_entry_in_split_mode(monkeypatch):
    """The allocation-free entry point runs the same rule: split-mode calls
    (the library's scratch array as the workspace) match the caller-workspace
    entry point bitwise, on a large call and then a smaller one."""
    import l20_pd_cabi as cabi
    from test_zz_no_alloc import run_noalloc

    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    big = H.make_synthetic(8, 28, 4, 128, [5000, 17, 1025, 3000, 512, 4097, 64, 2048], seed=81)
    small = H.make_synthetic(3, 16, 2, 128, [1700, 100, 1033], seed=82)
    for inp, split in ((big, 1024), (small, 512)):
        print("noalloc split-mode case", inp["query"].shape, split, flush=True)
        want = H.run_op(inp, split, via="cabi")
        got = run_noalloc(inp, split)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        H.compare(*got, *H.run_oracle(inp))


def test_library_takes_the_split_mode_at_256_token_splits(monkeypatch):
    """8 x 2048 tokens, 28 query / 4 KV heads: 256 triples at 256-token splits
    (one fp8 block per wave), the library's split; against the oracle."""
    import l20_pd_cabi as cabi

    monkeypatch.delenv("L20_PD_FUSED_SPLIT", raising=False)
    inp = H.make_synthetic(8, 28, 4, 128, [2048, 2000, 1100, 2048, 1500, 2048, 1777, 2040], per_head=True, seed=29)
    split = int(cabi.load().l20_pd_default_split_size(8, 4, inp["max_seq_len"], 0))
    assert split == 256
    out, lse, path = _run(inp, split, torch.float16)
    assert path == 2
    H.compare(out, lse, *H.run_oracle(inp))
