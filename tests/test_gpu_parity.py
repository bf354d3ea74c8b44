"""GPU parity: the HIP kernels against the CPU oracle on identical bytes.

Every test calls the library either through the torch dispatcher
(``torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out``) or straight through
the C ABI (ctypes).  Tolerances are the ones in ``pd_helpers``.
"""

import zlib

import numpy as np
import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    import l20_paged_decode  # noqa: F401  (fails loudly if the extension is missing)


# ------------------------------------------------------------ conversions
def test_fp8_conversions_match_oracle_table_on_all_codes():
    from oracle import paged_fp8_decode_ref as ref
    import l20_pd_cabi as cabi

    lib = cabi.load()
    codes = torch.arange(256, dtype=torch.uint8).repeat(3).cuda()  # 768: exercises the 4-byte tail
    codes = torch.cat([codes, codes[:3]])
    f32 = torch.empty(codes.numel(), dtype=torch.float32, device="cuda")
    bf = torch.empty(codes.numel(), dtype=torch.int16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert lib.l20_pd_fp8_e4m3_dequant_f32(codes.data_ptr(), f32.data_ptr(), codes.numel(), 1.0, s) == 0
    assert lib.l20_pd_fp8_e4m3_dequant_bf16(codes.data_ptr(), bf.data_ptr(), codes.numel(), s) == 0
    torch.cuda.synchronize()
    table = ref.e4m3fn_decode_table()
    want = table[codes.cpu().numpy()]
    got = f32.cpu().numpy()
    got_bf = bf.cpu().view(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    for g in (got, got_bf):
        assert np.array_equal(np.isnan(g), nan)
        assert np.array_equal(g[~nan], want[~nan])
        assert np.array_equal(np.signbit(g[~nan]), np.signbit(want[~nan]))
    # scaled dequantisation is code * scale in fp32
    assert lib.l20_pd_fp8_e4m3_dequant_f32(codes.data_ptr(), f32.data_ptr(), codes.numel(), 0.37, s) == 0
    torch.cuda.synchronize()
    scaled = f32.cpu().numpy()
    assert np.array_equal(scaled[~nan], (want[~nan] * np.float32(0.37)).astype(np.float32))


# ------------------------------------------------------------ the five configurations
CONFIG_SPLITS = {
    "c1_qwen2.5_0.5b": [64, 512],
    "c2_qwen2.5_coder_3b": [128, 256, 1024],  # 128: the library default
    "c3_qwen2.5_7b": [512, 1024],
    "c4_llama3_8b_long": [1024],
    # 1024 is the library default for this shape (the two-tile, one-block-in-
    # flight kernel on a fully static grid) and the split the bench measures
    "c5_llama3_70b_verify": [512, 1024],
}
# Sequences of config 5 checked against the oracle: 16 of 64, first and last
# included (each sequence's 4 rows x 8 query heads fill both 16-column query
# tiles of every KV head).
ORACLE_ROWS = {"c5_llama3_70b_verify": [0, 1, 5, 9, 17, 22, 28, 31, 32, 40, 45, 50, 55, 59, 62, 63]}


@pytest.mark.parametrize("name", list(CONFIG_SPLITS))
def test_config_parity(name):
    import l20_pd_workloads as wl

    cfg = wl.CONFIGS[name]
    inp = wl.make_inputs(cfg, device="cuda")
    inp["query"] = inp["query"].contiguous()
    rows_b = ORACLE_ROWS.get(name)
    exp_out, exp_lse = H.run_oracle(inp, rows=rows_b)
    rows = None
    if rows_b is not None:
        rows = np.concatenate([np.arange(b * cfg.q_len, (b + 1) * cfg.q_len) for b in rows_b])
    for split in CONFIG_SPLITS[name]:
        out, lse = H.run_op(inp, split)
        res = H.compare(out, lse, exp_out, exp_lse, rows=rows)
        print(name, split, res, flush=True)


# ------------------------------------------------------------ reference's own shapes
# vllm-main-l20-paged-decode-rfc.patch:487-582 (upstream test), seed 17, D=128
UPSTREAM = [(1, 129, 12, 2), (1, 2304, 16, 8), (4, 513, 12, 2), (4, 640, 16, 8)]


@pytest.mark.parametrize("batch,ctx,hq,hkv", UPSTREAM)
@pytest.mark.parametrize("split", [64, 128, 512])
def test_reference_upstream_shapes(batch, ctx, hq, hkv, split):
    inp = H.make_synthetic(batch, hq, hkv, 128, [ctx] * batch, seed=17)
    exp = H.run_oracle(inp)
    H.compare(*H.run_op(inp, split), *exp)


# ------------------------------------------------------------ edge cases
EDGE = [
    # batch, hq, hkv, d, lens, q_len, per_head, dtype
    ("ragged_d64", 5, 14, 2, 64, [1, 15, 16, 17, 500], 1, False, torch.bfloat16),
    ("ragged_d128", 5, 28, 4, 128, [1, 15, 16, 33, 1025], 1, True, torch.bfloat16),
    ("empty_seq", 3, 8, 2, 128, [0, 40, 0], 1, False, torch.bfloat16),
    ("fp16_query", 2, 16, 2, 128, [300, 77], 1, False, torch.float16),
    ("mha_g1", 2, 4, 4, 128, [200, 90], 1, False, torch.bfloat16),
    ("group16", 2, 32, 2, 128, [129, 700], 1, False, torch.bfloat16),
    ("verify_q4", 3, 16, 2, 128, [70, 4, 513], 4, False, torch.bfloat16),
    ("verify_q4_short", 2, 8, 2, 64, [2, 3], 4, True, torch.bfloat16),
    ("verify_q2_g16", 2, 32, 2, 128, [65, 300], 2, False, torch.bfloat16),
]


@pytest.mark.parametrize("case", EDGE, ids=[e[0] for e in EDGE])
@pytest.mark.parametrize("split", [64, 96, 1024])
def test_edge_cases(case, split):
    _, batch, hq, hkv, d, lens, q_len, per_head, dtype = case
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, dtype=dtype,
                           seed=zlib.crc32(case[0].encode()) % 1000, garbage_tail=True)
    exp = H.run_oracle(inp)
    H.compare(*H.run_op(inp, split), *exp)


# ------------------------------------------------------------ pages of 16 m tokens
PAGED = [
    # name, batch, hq, hkv, d, lens, q_len, per_head
    ("ragged", 5, 28, 4, 128, [1, 100, 333, 1024, 47], 1, True),
    ("empty_and_short", 4, 16, 2, 64, [0, 15, 16, 65], 1, False),
    ("verify_q4", 3, 16, 2, 128, [70, 4, 2049], 4, False),
]


@pytest.mark.parametrize("case", PAGED, ids=[c[0] for c in PAGED])
@pytest.mark.parametrize("page", [32, 48, 64])
@pytest.mark.parametrize("split", [64, 256, 1024])
def test_pages_of_a_multiple_of_16_tokens(case, page, split):
    """Caches of page-token pages (the reference hook's ``token // page_size``
    gather, integrations/vllm/l20_paged_split_kv.py:182-200), bytes past each
    sequence's end NaN: the torch op and the C ABI against the oracle."""
    name, batch, hq, hkv, d, lens, q_len, per_head = case
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, page=page,
                           seed=zlib.crc32(name.encode()) % 1000 + page, garbage_tail=True)
    assert inp["key_cache"].shape[1] == page
    exp = H.run_oracle(inp)
    H.compare(*H.run_op(inp, split, via="torch"), *exp)
    H.compare(*H.run_op(inp, split, via="cabi", partial_dtype=torch.float16), *exp)


@pytest.mark.parametrize("csr", [False, True], ids=["table", "csr"])
@pytest.mark.parametrize("page", [32, 64])
def test_16bit_kv_pages_of_a_multiple_of_16_tokens(csr, page):
    inp = H.make_synthetic16(4, 16, 2, 128, [1, 300, 1000, 64], dtype=torch.bfloat16, seed=page, page=page,
                             csr_pad=2, garbage_tail=True)
    H.compare(*H.run_op16(inp, 256, csr=csr), *H.run_oracle16(inp, csr=csr))


def test_hook_api_passes_the_block_size_through():
    import l20_paged_split_kv as hook

    inp = H.make_synthetic(3, 28, 4, 128, [900, 31, 2500], seed=8, page=64)
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    hook.l20_paged_split_kv_attention_fp8(q, inp["key_cache"], inp["value_cache"], inp["block_table"],
                                          inp["seq_lens"], output=out, k_scale=inp["k_scale"],
                                          v_scale=inp["v_scale"], lse=lse)
    H.compare(out, lse, *H.run_oracle(inp))
    # every other token row of a wider buffer: still one token stride per page, read right
    wide = torch.zeros(inp["key_cache"].shape[0], 128, 4, 128, dtype=torch.uint8, device=q.device)
    wide[:, ::2] = inp["key_cache"].view(torch.uint8)
    wide_v = torch.zeros_like(wide)
    wide_v[:, ::2] = inp["value_cache"].view(torch.uint8)
    out2 = torch.empty_like(q)
    hook.l20_paged_split_kv_attention_fp8(q, wide[:, ::2].view(inp["key_cache"].dtype),
                                          wide_v[:, ::2].view(inp["key_cache"].dtype), inp["block_table"],
                                          inp["seq_lens"], output=out2, k_scale=inp["k_scale"],
                                          v_scale=inp["v_scale"])
    assert torch.equal(out2, out)
    # padded pages (page stride != 64 token strides) are refused, not misread
    padded = torch.zeros(inp["key_cache"].shape[0], 80, 4, 128, dtype=inp["key_cache"].dtype,
                         device=q.device)[:, :64]
    with pytest.raises(RuntimeError):
        hook.l20_paged_split_kv_attention_fp8(q, padded, padded, inp["block_table"], inp["seq_lens"],
                                              output=out, k_scale=inp["k_scale"], v_scale=inp["v_scale"])


def test_c_abi_and_torch_op_agree_bitwise():
    inp = H.make_synthetic(3, 28, 4, 128, [900, 31, 4000], seed=5)
    a = H.run_op(inp, 256, via="torch")
    b = H.run_op(inp, 256, via="cabi")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    H.compare(*b, *H.run_oracle(inp))


def test_fp16_partial_workspace():
    inp = H.make_synthetic(2, 16, 2, 128, [1500, 700], seed=6)
    H.compare(*H.run_op(inp, 128, partial_dtype=torch.float16), *H.run_oracle(inp))


@pytest.mark.parametrize("d,lens,split,pdt", [
    (64, [8000, 3000, 1], 64, torch.float32),     # 125 splits: 4 waves per merged pair
    (128, [6000, 0, 700], 64, torch.float16),     # 94 splits: 8 waves per pair, fp16 partials
    (128, [8300, 10, 4000], 64, torch.bfloat16),  # 130 splits: 16 waves per pair, bf16 partials
    (128, [2100, 1000], 160, torch.float32),      # 14 splits: 1 wave per pair
])
def test_merge_waves_per_pair(d, lens, split, pdt):
    """The merge spreads a row's splits over 1-16 waves (each wave takes up to
    four steps of 512/D slots); every spread matches the oracle.  All four cases
    also take the speculative first-group loads (workspaces under 4 MB with
    slots past the first step)."""
    inp = H.make_synthetic(len(lens), 16, 2, d, lens, seed=split + d)
    H.compare(*H.run_op(inp, split, partial_dtype=pdt), *H.run_oracle(inp))


@pytest.mark.parametrize("d,lens,split,pdt", [
    (128, [4096, 4000, 1030, 5, 0], 1024, torch.float32),   # 4 slots, ragged rows
    (64, [511, 300, 64, 1], 64, torch.float16),              # 8 slots (the narrow limit), fp16 partials
    (128, [900, 2000], 256, torch.float32),                  # 8 slots, q_len 4 below
    (128, [2048, 1500, 3, 0], 1024, torch.bfloat16),         # 2 slots, bf16 partials
    (128, [1536, 700], 512, torch.float16),                  # 3 splits read as 4 slots (slot 3 rereads 0)
    (64, [300, 129, 64], 64, torch.bfloat16),                # 5 splits read as 8 slots, bf16 partials
])
@pytest.mark.parametrize("q_len", [1, 4])
def test_narrow_merge_ignores_stale_slots(d, lens, split, pdt, q_len):
    """With at most 8 split slots and at least 4096 (row, head) pairs the merge
    reads every slot with the length; slots past a row's split count hold
    NaN / inf from an earlier call and must not count."""
    import l20_pd_cabi as cabi

    # 64 query heads: batch x q_len x 64 >= 4096 pairs for the narrow merge once
    # the batch is filled up with short sequences (cheap for the oracle)
    batch = 4096 // (64 * q_len)
    lens = lens + [(37 * i) % 200 + q_len for i in range(batch - len(lens))]
    inp = H.make_synthetic(batch, 64, 8, d, lens, q_len=q_len, seed=split + d + q_len)
    po, pm, ps = H.workspace(inp, split, pdt)
    for t, v in ((po, float("nan")), (pm, float("inf")), (ps, float("nan"))):
        t.fill_(v)
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                  po, pm, ps, out, inp["k_scale"], inp["v_scale"], inp["max_seq_len"], split,
                                  softmax_scale=inp["softmax_scale"], q_len=q_len, lse=lse)
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    H.compare(out, lse, *H.run_oracle(inp))


@pytest.mark.parametrize("pdt", [torch.float32, torch.float16, torch.bfloat16])
def test_speculative_merge_loads_ignore_slots_past_each_row(pdt):
    """A small workspace with more slots than a wave's first step (here 30
    slots of 128 tokens, two waves per pair) is merged with every slot of the
    first step group loaded before the row's split count is known: slots
    past a row's count hold NaN / +inf and must not count, for rows of one
    split up to the whole workspace."""
    import l20_pd_cabi as cabi

    lens = [3840, 1, 129, 0, 1000, 3000, 257, 640]
    inp = H.make_synthetic(len(lens), 16, 2, 128, lens, seed=77)
    po, pm, ps = H.workspace(inp, 128, pdt)
    assert po.shape[2] == 30
    for t, v in ((po, float("nan")), (pm, float("inf")), (ps, float("nan"))):
        t.fill_(v)
    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                  po, pm, ps, out, inp["k_scale"], inp["v_scale"], inp["max_seq_len"], 128,
                                  softmax_scale=inp["softmax_scale"], lse=lse)
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    H.compare(out, lse, *H.run_oracle(inp))


def test_launches_on_two_streams_overlap_safely():
    """Two calls in flight on one device (two streams, each with its own
    workspace) use different work-queue counters: results are bitwise those
    of the calls run one at a time.  (The argument structs keep their
    workspaces alive: the loop below rebinds the names.)"""
    import l20_pd_cabi as cabi

    cases = [H.make_synthetic(16, 16, 2, 128, [3000 - 97 * i for i in range(16)], seed=71),
             H.make_synthetic(24, 28, 4, 128, [1500 + 61 * i for i in range(24)], seed=72)]
    calls = []
    for inp in cases:
        po, pm, ps = H.workspace(inp, 256)
        out = torch.empty_like(inp["query"])
        lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
        args = cabi.args_from_tensors(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                      inp["seq_lens"], po, pm, ps, out, inp["k_scale"], inp["v_scale"],
                                      inp["max_seq_len"], 256, softmax_scale=inp["softmax_scale"], lse=lse)
        calls.append((args, out, lse))
    serial = []
    for args, out, lse in calls:
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        serial.append((out.clone(), lse.clone()))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(20):
        for (args, _, _), s in zip(calls, streams):
            cabi.split_out(args, s.cuda_stream)
    torch.cuda.synchronize()
    for (_, out, lse), (s_out, s_lse) in zip(calls, serial):
        assert torch.equal(out, s_out) and torch.equal(lse, s_lse)
    for inp, (out, lse) in zip(cases, serial):
        H.compare(out, lse, *H.run_oracle(inp))


def test_two_streams_at_headline_scale():
    """Two config-3 calls (different input sets) in flight on two streams, ten
    rounds: both drain real work queues at once (claims, pre-assigned items,
    counter resets on different slots); results are bitwise the serial ones."""
    import l20_pd_cabi as cabi
    import l20_pd_workloads as wl

    cfg = wl.CONFIGS["c3_qwen2.5_7b"]
    sets = [wl.make_inputs(cfg, device="cuda", seed=cfg.seed + 500 + i) for i in range(2)]
    max_seq = max(s["max_seq_len"] for s in sets)
    calls = []
    for s in sets:
        po, pm, ps = H.workspace(dict(s, max_seq_len=max_seq), 512)
        out = torch.empty_like(s["query"])
        lse = torch.empty(s["query"].shape[:2], dtype=torch.float32, device="cuda")
        args = cabi.args_from_tensors(s["query"], s["key_cache"], s["value_cache"], s["block_table"], s["seq_lens"],
                                      po, pm, ps, out, s["k_scale"], s["v_scale"], max_seq, 512,
                                      softmax_scale=s["softmax_scale"], lse=lse)
        calls.append((args, out, lse))
    serial = []
    for args, out, lse in calls:
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        serial.append((out.clone(), lse.clone()))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(10):
        for (args, _, _), st in zip(calls, streams):
            cabi.split_out(args, st.cuda_stream)
        torch.cuda.synchronize()
        for (_, out, lse), (s_out, s_lse) in zip(calls, serial):
            assert torch.equal(out, s_out) and torch.equal(lse, s_lse)
    # and the serial results are right (a sample of rows against the oracle)
    rows = [0, 17, 64, 127]
    for s, (out, lse) in zip(sets, serial):
        H.compare(out, lse, *H.run_oracle(s, rows=rows), rows=rows)


HOSTILE = [
    # name, batch, hq, hkv, d, lens, max_wg (0: the full persistent grid)
    ("all_static_items", 16, 16, 2, 128, [3000 - 97 * i for i in range(16)], 0),
    ("queue_items", 24, 28, 4, 128, [1500 + 61 * i for i in range(24)], 5),
    ("one_split_rows", 6, 16, 2, 128, [3000, 1, 256, 0, 257, 40], 0),
]


@pytest.mark.parametrize("case", HOSTILE, ids=[c[0] for c in HOSTILE])
def test_results_do_not_depend_on_prior_buffer_contents(case, monkeypatch):
    """Workspace, output and LSE buffers come from ``torch.empty``: whatever a
    call reads it has written itself, so NaN, infinite or huge prior contents
    (including +inf in slot 0, the merge's "already final" marker) change
    nothing, bitwise."""
    import l20_pd_cabi as cabi

    name, batch, hq, hkv, d, lens, max_wg = case
    if max_wg:
        monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", str(max_wg))
    inp = H.make_synthetic(batch, hq, hkv, d, lens, seed=zlib.crc32(name.encode()) % 1000)
    exp = H.run_oracle(inp)
    po, pm, ps = H.workspace(inp, 256, extra_splits=2)
    out = torch.empty_like(inp["query"])
    lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
    args = cabi.args_from_tensors(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                  inp["seq_lens"], po, pm, ps, out, inp["k_scale"], inp["v_scale"],
                                  inp["max_seq_len"], 256, softmax_scale=inp["softmax_scale"], lse=lse)
    first = None
    for fill in (float("nan"), float("inf"), float("-inf"), 3e38, -3e38, 0.0):
        for t in (po, pm, ps, lse):
            t.fill_(fill)
        out.fill_(fill if fill == fill and abs(fill) < 1e38 else 0.0)
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        H.compare(out, lse, *exp)
        if first is None:
            first = (out.clone(), lse.clone())
        else:
            assert torch.equal(out, first[0]) and torch.equal(lse, first[1]), f"prior contents {fill} changed the result"


def test_strided_kv_views_like_vllm_unbind():
    """vLLM's cache is [num_blocks, 2, 16, Hkv, D]; unbind(1) gives strided K/V views."""
    inp = H.make_synthetic(3, 16, 8, 128, [100, 1000, 37], seed=7)
    joint = torch.stack([inp["key_cache"], inp["value_cache"]], dim=1)  # [P, 2, 16, Hkv, D]
    k_view, v_view = joint.unbind(1)
    assert k_view.stride(0) == 2 * 16 * 8 * 128
    out = H.run_op(inp, 128, key_cache=k_view, value_cache=v_view)
    H.compare(*out, *H.run_oracle(inp))


def test_split_size_invariance():
    inp = H.make_synthetic(4, 28, 4, 128, [5000, 1234, 77, 2048], seed=8)
    exp = H.run_oracle(inp)
    outs = []
    for split in (64, 128, 272, 512, 1024):
        out, lse = H.run_op(inp, split)
        H.compare(out, lse, *exp)
        outs.append(out.float())
    for o in outs[1:]:
        assert float((o - outs[0]).abs().max()) <= 1e-2


def test_hook_api_with_auto_split_and_reused_workspace():
    import l20_paged_split_kv as sk

    inp = H.make_synthetic(8, 16, 2, 128, [600, 2048, 31, 4096, 1, 300, 999, 2500], seed=9, per_head=True)
    ws = sk.allocate_l20_paged_split_kv_workspace(inp["query"], inp["max_seq_len"], split_size=256)
    exp = H.run_oracle(inp)
    for _ in range(2):
        lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
        out = sk.l20_paged_split_kv_attention_fp8(
            inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
            k_scale=inp["k_scale"], v_scale=inp["v_scale"], max_seq_len=inp["max_seq_len"], split_size=256,
            workspace=ws, lse=lse)
        torch.cuda.synchronize()
        H.compare(out, lse, *exp)
    out = sk.l20_paged_split_kv_attention_fp8(
        inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
        k_scale=inp["k_scale"], v_scale=inp["v_scale"], split_size=None)
    torch.cuda.synchronize()
    H.compare(out, None, exp[0], None, check_lse=False)


@pytest.mark.parametrize("max_wg", [0, 5], ids=["static_grid", "queue"])
def test_hip_graph_capture_replays_match_eager(max_wg, monkeypatch):
    """Replays reuse the captured launch's work-queue slot: with a 5-workgroup
    grid every replay drains a queue and must find its counter reset by the
    previous replay's last claim."""
    import l20_paged_decode  # noqa: F401

    if max_wg:
        monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", str(max_wg))
    inp = H.make_synthetic(4, 28, 4, 128, [3000, 700, 64, 1500], seed=10)
    po, pm, ps = H.workspace(inp, 256)
    out = torch.empty_like(inp["query"])
    lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")

    def call():
        torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
            inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
            po, pm, ps, out, inp["k_scale"], inp["v_scale"], inp["max_seq_len"], 256,
            inp["softmax_scale"], None, None, 1, lse)

    call()
    torch.cuda.synchronize()
    eager_out, eager_lse = out.clone(), lse.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(4):
        out.zero_()
        lse.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out) and torch.equal(lse, eager_lse)
    H.compare(eager_out, eager_lse, *H.run_oracle(inp))


def test_queue_counters_reset_across_slot_reuse(monkeypatch):
    """150 back-to-back queue-driven launches on one stream share the stream's
    work-queue slot; each launch must start on a counter the previous launch
    reset (a stale counter would skip items and change the result)."""
    import l20_pd_cabi as cabi

    monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", "7")
    inp = H.make_synthetic(6, 16, 2, 128, [2100, 17, 900, 0, 1300, 64], seed=12)
    exp = H.run_oracle(inp)
    po, pm, ps = H.workspace(inp, 64)
    out = torch.empty_like(inp["query"])
    lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
    args = cabi.args_from_tensors(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                  inp["seq_lens"], po, pm, ps, out, inp["k_scale"], inp["v_scale"],
                                  inp["max_seq_len"], 64, softmax_scale=inp["softmax_scale"], lse=lse)
    stream = torch.cuda.current_stream().cuda_stream
    cabi.split_out(args, stream)
    torch.cuda.synchronize()
    H.compare(out, lse, *exp)
    first = (out.clone(), lse.clone())
    outs = torch.empty((150,) + tuple(out.shape), dtype=out.dtype, device="cuda")
    lses = torch.empty((150,) + tuple(lse.shape), dtype=lse.dtype, device="cuda")
    for i in range(150):
        cabi.split_out(args, stream)
        outs[i].copy_(out)
        lses[i].copy_(lse)
    torch.cuda.synchronize()
    bad = [i for i in range(150) if not (torch.equal(outs[i], first[0]) and torch.equal(lses[i], first[1]))]
    assert not bad, f"launches {bad[:10]} differ from the first"


# ------------------------------------------------------------ work queue
# L20_PD_MAX_WORKGROUPS caps the persistent grid, so each workgroup streams
# many items (and unit-to-unit prefetch crosses items of different sequences).
# With items left over, workgroups [G/2, G) start on pre-assigned items of the
# compact numbering: grids of 2, 3 and 5 put 1, 1 and 2 workgroups there.
QUEUE = [
    # name, batch, hq, hkv, d, lens, q_len, split
    ("compact_ragged", 8, 16, 2, 128, [3000, 0, 17, 700, 64, 1, 2049, 333], 1, 64),
    ("two_heads_per_wave", 3, 24, 12, 128, [900, 31, 400], 1, 128),
    ("three_heads_per_wave_d64", 2, 18, 9, 64, [500, 77], 1, 64),
    ("verify_q4", 4, 16, 2, 128, [700, 4, 130, 1500], 4, 96),
    # splits of 1024 tokens: the one-block-in-flight stream (fp8, head_dim 128)
    ("long_units_one_block", 4, 16, 2, 128, [5000, 33, 2048, 1100], 1, 1024),
    ("long_units_verify_q4", 3, 32, 4, 128, [3000, 1030, 5], 4, 1024),
    # more sequences than the LDS prefix holds: split-major numbering with holes
    ("split_major_fallback", 600, 4, 1, 64, None, 1, 64),
]


@pytest.mark.parametrize("case", QUEUE, ids=[c[0] for c in QUEUE])
@pytest.mark.parametrize("max_wg", [1, 2, 3, 5, 0])
def test_work_queue_small_grids(case, max_wg, monkeypatch):
    name, batch, hq, hkv, d, lens, q_len, split = case
    if lens is None:
        lens = np.random.default_rng(11).integers(0, 200, size=batch).tolist()
        lens[5] = 0
    if max_wg:
        monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", str(max_wg))
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, seed=zlib.crc32(name.encode()) % 1000,
                           garbage_tail=True)
    exp = H.run_oracle(inp)
    for _ in range(2):  # the queue counters reset themselves between launches
        H.compare(*H.run_op(inp, split), *exp)


# ------------------------------------------------------------ fp16/bf16-KV siblings (block table and CSR)
# The reference benchmark's shapes (benchmark_cuda_paged_decode.py:63-101): batch 1/4,
# contexts 512/2048/4096, fp16, 128-dim heads.
SIB_REF = [(1, 512), (4, 2048), (4, 4096)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("batch,ctx", SIB_REF)
@pytest.mark.parametrize("csr", [False, True], ids=["table", "csr"])
def test_16bit_kv_reference_shapes(dtype, batch, ctx, csr):
    inp = H.make_synthetic16(batch, 32, 8, 128, [ctx] * batch, dtype=dtype, seed=ctx + batch, csr_pad=2)
    exp = H.run_oracle16(inp, csr=csr)
    H.compare(*H.run_op16(inp, 512, csr=csr), *exp)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_allocating_entry_points_match_the_oracle(dtype):
    """paged_decode and paged_decode_split, the reference extension's allocating
    entry points (l20_paged_decode.cu:467-547), on its benchmark's head layout
    (16 query heads, 8 KV heads, head_dim 128) with ragged lengths: each returns
    a new output that matches the oracle; paged_decode takes its split size from
    the block table's bound."""
    import l20_paged_decode as ext

    inp = H.make_synthetic16(4, 16, 8, 128, [512, 2048, 1, 700], dtype=dtype, seed=91)
    exp_out, _ = H.run_oracle16(inp)
    args = (inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"])
    outs = [ext.paged_decode(*args)] + [ext.paged_decode_split(*args, inp["max_seq_len"], s) for s in (64, 128, 512)]
    torch.cuda.synchronize()
    for out in outs:
        assert out.dtype == dtype and out.shape == inp["query"].shape
        H.compare(out, None, exp_out, None)


SIB_EDGE = [
    # name, batch, hq, hkv, d, lens, q_len
    ("ragged_d128", 5, 28, 4, 128, [1, 15, 16, 33, 1025], 1),
    ("ragged_d64", 4, 14, 2, 64, [0, 40, 511, 17], 1),
    ("mha", 2, 4, 4, 128, [200, 90], 1),
    ("group16_verify_q2", 2, 32, 2, 128, [65, 300], 2),
    ("verify_q4", 3, 16, 2, 128, [70, 4, 513], 4),
]


@pytest.mark.parametrize("case", SIB_EDGE, ids=[c[0] for c in SIB_EDGE])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("split", [64, 1024])
def test_16bit_kv_edge_cases(case, dtype, split):
    name, batch, hq, hkv, d, lens, q_len = case
    inp = H.make_synthetic16(batch, hq, hkv, d, lens, dtype=dtype, q_len=q_len, garbage_tail=True,
                             seed=zlib.crc32(name.encode()) % 1000, csr_pad=1)
    exp = H.run_oracle16(inp)
    H.compare(*H.run_op16(inp, split), *exp)
    H.compare(*H.run_op16(inp, split, csr=True, via="cabi"), *exp)


def test_16bit_kv_fp16_partials_and_small_grid(monkeypatch):
    monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", "3")
    inp = H.make_synthetic16(6, 16, 2, 128, [3000, 0, 17, 700, 64, 1], dtype=torch.float16, seed=44)
    exp = H.run_oracle16(inp)
    for _ in range(2):
        H.compare(*H.run_op16(inp, 64, partial_dtype=torch.float16), *exp)


def test_fp8_op_rejects_16bit_caches_and_vice_versa():
    inp = H.make_synthetic16(2, 8, 2, 128, [40, 20], dtype=torch.float16, seed=1)
    po, pm, ps = H.workspace(inp, 64)
    out = torch.empty_like(inp["query"])
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
            inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"], po, pm, ps, out,
            1.0, 1.0, inp["max_seq_len"], 64)
    fp8 = H.make_synthetic(2, 8, 2, 128, [40, 20], seed=1)
    with pytest.raises(RuntimeError, match="query's dtype"):
        torch.ops.l20_stack.paged_decode_split_out(
            fp8["query"], fp8["key_cache"], fp8["value_cache"], fp8["block_table"], fp8["seq_lens"], po, pm, ps,
            torch.empty_like(fp8["query"]), fp8["max_seq_len"], 64)


# ------------------------------------------------------------ OCP e5m2 caches
# The reference's hook-facing Triton op accepts float8_e5m2 caches
# (integrations/vllm/l20_paged_split_kv.py:617-621) and dequantises them as
# code * scale like e4m3fn ones.
E5M2 = [
    # name, batch, hq, hkv, d, lens, q_len, per_head, dtype
    ("ragged_d128", 5, 28, 4, 128, [1, 15, 16, 33, 1025], 1, False, torch.bfloat16),
    ("ragged_d64_per_head", 5, 14, 2, 64, [1, 15, 16, 17, 500], 1, True, torch.float16),
    ("empty_seq", 3, 8, 2, 128, [0, 40, 0], 1, False, torch.bfloat16),
    ("verify_q4", 3, 16, 2, 128, [70, 4, 513], 4, False, torch.bfloat16),
    ("long_gqa7", 2, 28, 4, 128, [4096, 2500], 1, False, torch.bfloat16),
]


@pytest.mark.parametrize("case", E5M2, ids=[c[0] for c in E5M2])
@pytest.mark.parametrize("split", [64, 512])
@pytest.mark.parametrize("via", ["torch", "cabi"])
def test_e5m2_caches(case, split, via):
    _, batch, hq, hkv, d, lens, q_len, per_head, dtype = case
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, dtype=dtype, fp8="e5m2",
                           seed=zlib.crc32(case[0].encode()) % 1000, garbage_tail=True)
    assert inp["key_cache"].dtype == torch.float8_e5m2
    exp = H.run_oracle(inp)
    H.compare(*H.run_op(inp, split, via=via), *exp)


def test_e5m2_every_finite_code_end_to_end():
    """V: 248 one-token sequences, sequence c's value row all code c: the output
    (fp16, which holds every e5m2 value) is the code's value exactly.  K: 248
    two-token sequences, key 0 = code c on dim 0, key 1 = 0, query = e_0 with
    softmax scale 1: the LSE is log(1 + exp(value(c)))."""
    from oracle import paged_fp8_decode_ref as ref

    table = ref.e5m2_decode_table()
    codes = np.array([c for c in range(256) if np.isfinite(table[c])], dtype=np.uint8)
    n, d = len(codes), 128
    assert n == 248
    vc = torch.zeros(n + 1, 16, 1, d, dtype=torch.uint8)
    vc[:n, 0, 0, :] = torch.from_numpy(codes)[:, None]
    kc = torch.zeros(n + 1, 16, 1, d, dtype=torch.uint8)
    kc[:n, 0, 0, 0] = torch.from_numpy(codes)
    vk = torch.zeros_like(vc)
    vk[:n, 0, 0, :] = 0x3C  # e5m2 1.0: out = softmax weight of key 0
    query = torch.zeros(n, 1, d, dtype=torch.float16)
    query[:, 0, 0] = 1.0
    table_t = torch.arange(n, dtype=torch.int32).view(n, 1)
    base = {"query": query.cuda(), "block_table": table_t.cuda(), "k_scale": 1.0, "v_scale": 1.0,
            "softmax_scale": 1.0, "q_len": 1}
    v_case = dict(base, key_cache=torch.zeros_like(vc).view(torch.float8_e5m2).cuda(),
                  value_cache=vc.view(torch.float8_e5m2).cuda(),
                  seq_lens=torch.ones(n, dtype=torch.int32).cuda(), max_seq_len=1)
    out, _ = H.run_op(v_case, 64)
    want = table[codes]
    got = out[:, 0, :].float().cpu().numpy()
    assert np.array_equal(got, np.broadcast_to(want[:, None], got.shape))
    k_case = dict(base, key_cache=kc.view(torch.float8_e5m2).cuda(), value_cache=vk.view(torch.float8_e5m2).cuda(),
                  seq_lens=torch.full((n,), 2, dtype=torch.int32).cuda(), max_seq_len=2)
    _, lse = H.run_op(k_case, 64)
    exact = np.logaddexp(table[codes].astype(np.float64), 0.0)
    got_lse = lse[:, 0].cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got_lse, exact, rtol=2e-6, atol=2e-5)


def test_e5m2_hook_api_and_noalloc():
    import l20_pd_cabi as cabi
    from l20_paged_split_kv import allocate_l20_paged_split_kv_workspace, l20_paged_split_kv_attention_fp8

    inp = H.make_synthetic(4, 28, 4, 128, [3000, 700, 64, 1500], fp8="e5m2", seed=33)
    exp = H.run_oracle(inp)
    ws = allocate_l20_paged_split_kv_workspace(inp["query"], inp["max_seq_len"], split_size=512)
    out = l20_paged_split_kv_attention_fp8(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                           inp["seq_lens"], k_scale=inp["k_scale"], v_scale=inp["v_scale"],
                                           max_seq_len=inp["max_seq_len"], split_size=512, workspace=ws)
    torch.cuda.synchronize()
    H.compare(out, None, exp[0], exp[1], check_lse=False)
    out2 = torch.empty_like(inp["query"])
    lse2 = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
    po, pm, ps = H.workspace(inp, 512)
    args = cabi.args_from_tensors(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                  inp["seq_lens"], po, pm, ps, out2, inp["k_scale"], inp["v_scale"],
                                  inp["max_seq_len"], 512, softmax_scale=inp["softmax_scale"], lse=lse2)
    assert args.kv_dtype == cabi.L20_PD_KV_FP8_E5M2
    cabi.split_out_noalloc(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    H.compare(out2, lse2, *exp)


def test_mixed_fp8_formats_are_rejected():
    inp = H.make_synthetic(2, 8, 2, 128, [40, 20], seed=1)
    v5 = inp["value_cache"].float().to(torch.float8_e5m2)
    po, pm, ps = H.workspace(inp, 64)
    with pytest.raises(RuntimeError, match="float8"):
        torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(
            inp["query"], inp["key_cache"], v5, inp["block_table"], inp["seq_lens"], po, pm, ps,
            torch.empty_like(inp["query"]), 1.0, 1.0, inp["max_seq_len"], 64)


# ------------------------------------------------------------ the reference allocator's workspace
def test_reference_allocator_workspace_bf16_partials():
    """A workspace laid out as the reference's allocate_l20_paged_split_kv_workspace
    makes it (integrations/vllm/l20_paged_split_kv.py:14-30: partial_output in the
    query dtype, next_pow2(ceil(max_seq_len / split)) splits) works as given."""
    from l20_paged_split_kv import l20_paged_split_kv_attention_fp8

    inp = H.make_synthetic(6, 28, 4, 128, [3000, 17, 700, 1, 1500, 2049], seed=61)
    exp = H.run_oracle(inp)
    q = inp["query"]
    n_s = 1 << (-(-inp["max_seq_len"] // 512) - 1).bit_length()  # next power of two: 6 -> 8
    assert n_s == 8
    ws = (torch.empty(q.shape[0], q.shape[1], n_s, 128, dtype=q.dtype, device="cuda"),
          torch.empty(q.shape[0], q.shape[1], n_s, device="cuda"),
          torch.empty(q.shape[0], q.shape[1], n_s, device="cuda"),
          torch.empty_like(q))
    out = l20_paged_split_kv_attention_fp8(q, inp["key_cache"], inp["value_cache"], inp["block_table"],
                                           inp["seq_lens"], k_scale=inp["k_scale"], v_scale=inp["v_scale"],
                                           max_seq_len=inp["max_seq_len"], split_size=512, workspace=ws)
    torch.cuda.synchronize()
    assert out.data_ptr() == ws[3].data_ptr()
    H.compare(out, None, exp[0], exp[1], check_lse=False)


@pytest.mark.parametrize("case", EDGE[:4], ids=[e[0] for e in EDGE[:4]])
@pytest.mark.parametrize("split", [64, 1024])
def test_bf16_partial_workspace(case, split):
    _, batch, hq, hkv, d, lens, q_len, per_head, dtype = case
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, per_head=per_head, dtype=dtype,
                           seed=zlib.crc32(case[0].encode()) % 1000 + 3, garbage_tail=True)
    H.compare(*H.run_op(inp, split, partial_dtype=torch.bfloat16), *H.run_oracle(inp))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_16bit_hook_facing_function(dtype):
    """l20_paged_split_kv_attention (the reference's 16-bit entry, l20_paged_split_kv.py:491-595):
    its keywords, a reused reference-shaped workspace, and the Triton-variant knobs accepted."""
    from l20_paged_split_kv import allocate_l20_paged_split_kv_workspace, l20_paged_split_kv_attention

    inp = H.make_synthetic16(5, 16, 2, 128, [2049, 1, 700, 0, 1300], dtype=dtype, seed=71)
    exp = H.run_oracle16(inp)
    ws = allocate_l20_paged_split_kv_workspace(inp["query"], inp["max_seq_len"], split_size=512)
    for kw in ({}, {"page_granular": True}, {"grouped_gqa": True}):
        out = l20_paged_split_kv_attention(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                           inp["seq_lens"], split_size=512, workspace=ws, **kw)
        torch.cuda.synchronize()
        H.compare(out, None, exp[0], exp[1], check_lse=False)
    with pytest.raises(RuntimeError, match="query's dtype"):
        l20_paged_split_kv_attention(inp["query"], inp["key_cache"].float(), inp["value_cache"].float(),
                                     inp["block_table"], inp["seq_lens"])
