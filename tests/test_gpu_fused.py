"""Single-launch path (GPU): one workgroup of 8 waves per (sequence, KV head),
each wave one eighth of the sequence, the waves' online-softmax states folded
in LDS; no split workspace is written and no merge kernel runs.

* Forced with L20_PD_FUSED=1 on every shape the path accepts (fp8 e4m3/e5m2
  and fp16/bf16 caches, block tables and CSR page lists, head_dim 64/128, one
  query tile incl. draft rows, ragged and empty rows, pages of 16/32/64
  tokens, per-head scales, sequences up to 8192 tokens):
  output and LSE against the oracle, through the torch op and the C ABI, and
  the workspace untouched (so the path that ran is the single launch).
* The library's own choice (the variable unset): the single launch at
  config 1 and for short sequences, the split kernels at config 2 (2048
  tokens per sequence), both against the oracle.
* Verification: draft rows (causal) and random ancestor trees over one and
  two query tiles, forced and by the library's choice.
* Sequences longer than the path covers run the split kernels even when it
  is asked for.
"""

import zlib

import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu

CASES = [
    # name, batch, hq, hkv, d, lens, q_len, per_head, fp8, page
    ("ragged_d128", 5, 28, 4, 128, [1, 15, 16, 33, 1025], 1, True, "e4m3fn", 16),
    ("ragged_d64", 5, 14, 2, 64, [1, 15, 16, 17, 500], 1, False, "e4m3fn", 16),
    ("empty_rows", 3, 8, 2, 128, [0, 40, 0], 1, False, "e4m3fn", 16),
    ("mha_g1", 2, 4, 4, 128, [200, 90], 1, False, "e4m3fn", 16),
    ("group16", 2, 32, 2, 128, [129, 700], 1, False, "e4m3fn", 16),
    ("verify_q4_g4", 3, 8, 2, 128, [70, 4, 513], 4, False, "e4m3fn", 16),
    ("verify_q2_g8_d64", 2, 16, 2, 64, [2, 300], 2, True, "e4m3fn", 16),
    ("long_8192", 2, 16, 2, 128, [8192, 5000], 1, False, "e4m3fn", 16),
    ("e5m2", 4, 16, 2, 128, [1, 333, 2048, 64], 1, True, "e5m2", 16),
    ("pages_32", 4, 16, 2, 128, [1, 100, 2049, 64], 1, False, "e4m3fn", 32),
    ("pages_64", 3, 28, 4, 128, [900, 31, 2500], 1, True, "e4m3fn", 64),
]


def _run_cabi(inp, split, pdt=torch.float32):
    """The C ABI with a NaN-filled workspace; returns (out, lse, workspace
    untouched)."""
    import l20_pd_cabi as cabi

    po, pm, ps = H.workspace(inp, split, pdt)
    for t in (po, pm, ps):
        t.fill_(float("nan"))
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    ks, ksph = H._scales(inp["k_scale"])
    vs, vsph = H._scales(inp["v_scale"])
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                  po, pm, ps, out, ks, vs, inp["max_seq_len"], split,
                                  softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], lse=lse,
                                  k_scale_per_head=ksph, v_scale_per_head=vsph, tree_mask=inp.get("tree_mask"))
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    untouched = bool(torch.isnan(pm).all() and torch.isnan(ps).all() and torch.isnan(po.float()).all())
    return out, lse, untouched


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_single_launch_matches_oracle(case, monkeypatch):
    name, batch, hq, hkv, d, lens, q_len, per_head, fp8, page = case
    monkeypatch.setenv("L20_PD_FUSED", "1")
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, fp8=fp8, page=page,
                           seed=zlib.crc32(name.encode()) % 1000, garbage_tail=True)
    exp = H.run_oracle(inp)
    H.compare(*H.run_op(inp, 512), *exp)
    for split, pdt in ((64, torch.float16), (1024, torch.float32)):
        out, lse, untouched = _run_cabi(inp, split, pdt)
        assert untouched, "the split workspace was written: the single launch did not run"
        H.compare(out, lse, *exp)


CASES16 = [
    # name, batch, hq, hkv, d, lens, q_len, dtype, page, csr
    ("fp16_ragged", 5, 28, 4, 128, [1, 15, 16, 33, 500], 1, torch.float16, 16, False),
    ("bf16_d64_q2", 3, 16, 2, 64, [2, 300, 0], 2, torch.bfloat16, 16, False),
    ("bf16_long_4096", 2, 16, 2, 128, [4096, 1000], 1, torch.bfloat16, 16, False),
    ("fp16_pages_32", 4, 16, 2, 128, [1, 100, 511, 64], 1, torch.float16, 32, False),
    ("bf16_csr", 4, 32, 8, 128, [1, 17, 480, 200], 1, torch.bfloat16, 16, True),
]


@pytest.mark.parametrize("case", CASES16, ids=[c[0] for c in CASES16])
def test_single_launch_16bit_caches(case, monkeypatch):
    """The same kernel over fp16/bf16 caches (16-token blocks): block tables
    and CSR page lists, against the oracle, the workspace untouched."""
    import l20_pd_cabi as cabi

    name, batch, hq, hkv, d, lens, q_len, dtype, page, csr = case
    monkeypatch.setenv("L20_PD_FUSED", "1")
    inp = H.make_synthetic16(batch, hq, hkv, d, lens, q_len=q_len, dtype=dtype, page=page, csr_pad=2,
                             seed=zlib.crc32(name.encode()) % 1000, garbage_tail=True)
    exp = H.run_oracle16(inp, csr=csr)
    po, pm, ps = H.workspace(inp, 256)
    for t in (po, pm, ps):
        t.fill_(float("nan"))
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    table = inp["page_indices"] if csr else inp["block_table"]
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], table, inp["seq_lens"], po, pm, ps, out,
                                  1.0, 1.0, inp["max_seq_len"], 256, softmax_scale=inp["softmax_scale"],
                                  q_len=q_len, lse=lse, page_indptr=inp["page_indptr"] if csr else None)
    assert cabi.single_launch(args)
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert bool(torch.isnan(pm).all() and torch.isnan(po.float()).all()), "the split workspace was written"
    H.compare(out, lse, *exp)
    H.compare(*H.run_op16(inp, 64, csr=csr), *exp)


@pytest.mark.parametrize("name,single", [("c1_qwen2.5_0.5b", True), ("c2_qwen2.5_coder_3b", False)])
def test_library_choice_at_configs_1_and_2(name, single, monkeypatch):
    import l20_pd_workloads as wl

    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    cfg = wl.CONFIGS[name]
    inp = wl.make_inputs(cfg, device="cuda")
    inp["query"] = inp["query"].contiguous()
    exp = H.run_oracle(inp)
    split = 128 if name.startswith("c2") else 64
    out, lse, untouched = _run_cabi(inp, split, torch.float16)
    assert untouched == single
    H.compare(out, lse, *exp)
    H.compare(*H.run_op(inp, split, partial_dtype=torch.float16), *exp)


def test_library_takes_the_single_launch_for_short_sequences(monkeypatch):
    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    inp = H.make_synthetic(64, 16, 2, 128, [1024 - 7 * i for i in range(64)], seed=5)
    out, lse, untouched = _run_cabi(inp, 128, torch.float16)
    assert untouched
    H.compare(out, lse, *H.run_oracle(inp))


TILES = [
    # name, batch, hq, hkv, d, lens, q_len, tree
    ("verify_2tiles", 4, 64, 8, 128, [1024, 17, 300, 4], 4, False),
    ("verify_2tiles_d64", 3, 32, 4, 64, [700, 64, 1], 4, False),
    ("tree_1tile", 3, 8, 2, 128, [700, 37, 1500], 4, True),
    ("tree_2tiles", 2, 16, 2, 128, [1000, 333], 4, True),
    ("tree_mha_d64", 2, 32, 32, 64, [530, 64], 8, True),
    ("tree_32drafts", 2, 4, 4, 128, [900, 32], 32, True),
]


@pytest.mark.parametrize("case", TILES, ids=[c[0] for c in TILES])
def test_single_launch_draft_rows_and_trees(case, monkeypatch):
    """Verification: draft rows under the causal rule or a random ancestor tree,
    one or two 16-column query tiles (fp16 fold slots for two), against the
    oracle; the workspace untouched."""
    import numpy as np
    from test_gpu_tree_verify import random_tree, words

    name, batch, hq, hkv, d, lens, q_len, tree = case
    monkeypatch.setenv("L20_PD_FUSED", "1")
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, seed=zlib.crc32(name.encode()) % 1000,
                           garbage_tail=True)
    if tree:
        rng = np.random.default_rng(zlib.crc32(name.encode()))
        inp["tree_mask"] = words(np.stack([random_tree(q_len, rng) for _ in range(batch)])).cuda()
    exp = H.run_oracle(inp)
    for split in (64, 1024):
        out, lse, untouched = _run_cabi(inp, split)
        assert untouched, "the split workspace was written: the single launch did not run"
        H.compare(out, lse, *exp)
    H.compare(*H.run_op(inp, 256, via="torch"), *exp)


def test_library_takes_the_single_launch_for_small_verify_batches(monkeypatch):
    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    inp = H.make_synthetic(16, 64, 8, 128, [512 - 9 * i for i in range(16)], q_len=4, seed=9)
    out, lse, untouched = _run_cabi(inp, 128)
    assert untouched
    H.compare(out, lse, *H.run_oracle(inp))


def test_sequences_beyond_the_single_launch_use_the_split_kernels(monkeypatch):
    monkeypatch.setenv("L20_PD_FUSED", "1")
    inp = H.make_synthetic(1, 16, 2, 128, [9000], seed=19)
    out, lse, untouched = _run_cabi(inp, 256, torch.float32)
    assert not untouched
    H.compare(out, lse, *H.run_oracle(inp))


def test_single_launch_graph_replays_match_eager(monkeypatch):
    """The single launch holds no state between calls: captured in a HIP graph
    and replayed three times, with eager calls between the replays, every
    replay is bitwise equal to the eager result."""
    import l20_pd_cabi as cabi

    monkeypatch.setenv("L20_PD_FUSED", "1")
    inp = H.make_synthetic(6, 28, 4, 128, [1000, 1, 517, 64, 0, 333], seed=12)
    po, pm, ps = H.workspace(inp, 256)
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                  po, pm, ps, out, inp["k_scale"], inp["v_scale"], inp["max_seq_len"], 256,
                                  softmax_scale=inp["softmax_scale"], lse=lse)
    assert cabi.single_launch(args)
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = (out.clone(), lse.clone())
    H.compare(out, lse, *H.run_oracle(inp))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
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


def test_noalloc_entry_takes_the_single_launch(monkeypatch):
    """The allocation-free entry point runs the same rule: a small batch takes
    the single launch (its scratch array is not needed) and matches the oracle
    and the allocating entry point bitwise."""
    import l20_pd_cabi as cabi

    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    inp = H.make_synthetic(5, 28, 4, 128, [1, 15, 16, 33, 1000], seed=31)
    exp = H.run_oracle(inp)
    q = inp["query"]
    outs = []
    for noalloc in (False, True):
        po, pm, ps = H.workspace(inp, 256)
        out = torch.empty_like(q)
        lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
        args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                      po, pm, ps, out, inp["k_scale"], inp["v_scale"], inp["max_seq_len"], 256,
                                      softmax_scale=inp["softmax_scale"], lse=lse)
        assert cabi.single_launch(args)
        (cabi.split_out_noalloc if noalloc else cabi.split_out)(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        H.compare(out, lse, *exp)
        outs.append((out, lse))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
