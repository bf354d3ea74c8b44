"""Robustness of the persistent partial kernel (GPU).

* Bounded hand-off waits: with a spin limit of one poll (set from the host
  with l20_pd_set_spin_limit) the waits between the waves of a workgroup give
  up at once; every kernel still exits normally, the give-up is reported through
  l20_pd_device_errors (with the queue-sharing error when a give-up left the
  work-queue counter mid-way), and after clearing, which also zeroes the
  counters, the next call is exact again.
* Counter slots: graph replays of a queue-driven call interleaved with eager
  queue-driven calls on another stream, each bitwise equal to its eager
  result (a graph's captured launch and the other stream's launches hold
  different work-queue slots).
* Counter sharing: two graphs captured 16 captures apart (one capture slot)
  replayed at the same time on two streams: every replay's results are
  bitwise exact, or the sharing is reported (L20_PD_DEVERR_QUEUE_SHARED), and
  after clearing, an eager call is exact again.
* Graph soak: one captured config-3 call replayed 1000 times, every replay
  bitwise equal to the eager call (the reference's stress of this op:
  scripts/stress_cuda_paged_decode.py:160-166, 1000 replays).
"""

from __future__ import annotations

import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu


def _call_args(inp, split, out, lse):
    import l20_pd_cabi as cabi

    po, pm, ps = H.workspace(inp, split)
    return cabi.args_from_tensors(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_table"],
                                  inp["seq_lens"], po, pm, ps, out, inp["k_scale"], inp["v_scale"],
                                  inp["max_seq_len"], split, softmax_scale=inp["softmax_scale"], lse=lse)


def test_hand_off_waits_give_up_and_report(monkeypatch):
    import l20_pd_cabi as cabi

    assert cabi.device_errors(clear=True) == 0, "a device error was pending before this test"
    inp = H.make_synthetic(8, 16, 2, 128, [3000, 0, 17, 700, 64, 1, 2049, 333], seed=21)
    exp = H.run_oracle(inp)
    out = torch.empty_like(inp["query"])
    lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
    # a 3-workgroup grid: every workgroup hands many items over between its waves
    monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", "3")
    cabi.set_spin_limit(1)
    try:
        args = _call_args(inp, 64, out, lse)
        for _ in range(3):
            cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    finally:
        cabi.set_spin_limit(0)
    err = cabi.device_errors(clear=False)
    # Wait give-ups (1, 2, 4).  A workgroup that gave up at the prefix wait
    # abandons a claim it had issued, so that launch never reaches its last
    # claim and leaves the counter mid-way: the next call reports
    # L20_PD_DEVERR_QUEUE_SHARED, and clearing zeroes the counter.
    assert err & 7 != 0 and err & ~(7 | cabi.L20_PD_DEVERR_QUEUE_SHARED) == 0, err
    assert cabi.device_errors(clear=True) == err
    assert cabi.device_errors() == 0
    # recovered: the same call with the normal limit is exact again
    out.zero_()
    lse.zero_()
    args = _call_args(inp, 64, out, lse)
    for _ in range(3):
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    H.compare(out, lse, *exp)
    assert cabi.device_errors() == 0


@pytest.mark.parametrize("value", [1 << 30, (0xDEADBEEF << 32) | 7])
def test_a_counter_left_in_use_is_reported_and_cleared(value, monkeypatch):
    """A work-queue counter that a launch left non-zero (a give-up mid-way, or
    two launches on one slot) is found by the next launch that claims: the
    call reports L20_PD_DEVERR_QUEUE_SHARED instead of silently skipping
    items, and after clearing the same call is exact again."""
    import l20_pd_cabi as cabi

    assert cabi.device_errors(clear=True) == 0, "a device error was pending before this test"
    lens = [1500 + 61 * i for i in range(24)]
    inp = H.make_synthetic(24, 28, 4, 128, lens, seed=23)
    exp = H.run_oracle(inp)
    out = torch.empty_like(inp["query"])
    lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
    # 5 workgroups for ~600 items: every launch claims from the counter
    monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", "5")
    args = _call_args(inp, 256, out, lse)
    cabi.set_queue_counters(value)
    try:
        cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert cabi.device_errors() == cabi.L20_PD_DEVERR_QUEUE_SHARED
    finally:
        cabi.device_errors(clear=True)
    assert cabi.device_errors() == 0
    out.zero_()
    lse.zero_()
    cabi.split_out(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    H.compare(out, lse, *exp)
    assert cabi.device_errors() == 0


def test_graph_replays_interleaved_with_eager_launches_on_another_stream(monkeypatch):
    import l20_pd_cabi as cabi

    monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", "5")  # both calls drain real work queues
    a = H.make_synthetic(4, 28, 4, 128, [3000, 700, 64, 1500], seed=10)
    b = H.make_synthetic(6, 16, 2, 128, [2100, 17, 900, 0, 1300, 64], seed=12)
    out_a = torch.empty_like(a["query"])
    lse_a = torch.empty(a["query"].shape[:2], dtype=torch.float32, device="cuda")
    out_b = torch.empty_like(b["query"])
    lse_b = torch.empty(b["query"].shape[:2], dtype=torch.float32, device="cuda")
    args_a = _call_args(a, 256, out_a, lse_a)
    args_b = _call_args(b, 64, out_b, lse_b)
    cabi.split_out(args_a, torch.cuda.current_stream().cuda_stream)
    cabi.split_out(args_b, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref_a = (out_a.clone(), lse_a.clone())
    ref_b = (out_b.clone(), lse_b.clone())
    H.compare(*ref_a, *H.run_oracle(a))
    H.compare(*ref_b, *H.run_oracle(b))

    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    sa.wait_stream(torch.cuda.current_stream())
    sb.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(sa):
        cabi.split_out(args_a, sa.cuda_stream)  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=sa):
            cabi.split_out(args_a, sa.cuda_stream)
    torch.cuda.synchronize()
    snaps_a = torch.empty((20,) + tuple(out_a.shape), dtype=out_a.dtype, device="cuda")
    snaps_b = torch.empty((20,) + tuple(out_b.shape), dtype=out_b.dtype, device="cuda")
    for i in range(20):
        with torch.cuda.stream(sa):
            graph.replay()
            snaps_a[i].copy_(out_a)
        with torch.cuda.stream(sb):
            cabi.split_out(args_b, sb.cuda_stream)
            cabi.split_out(args_b, sb.cuda_stream)
            snaps_b[i].copy_(out_b)
    torch.cuda.synchronize()
    bad_a = [i for i in range(20) if not torch.equal(snaps_a[i], ref_a[0])]
    bad_b = [i for i in range(20) if not torch.equal(snaps_b[i], ref_b[0])]
    assert not bad_a and not bad_b, (bad_a, bad_b)
    assert torch.equal(lse_a, ref_a[1]) and torch.equal(lse_b, ref_b[1])
    assert cabi.device_errors() == 0


def test_graphs_sharing_a_counter_slot_are_exact_or_reported(monkeypatch):
    import l20_pd_cabi as cabi

    assert cabi.device_errors(clear=True) == 0, "a device error was pending before this test"
    # A long queue-driven call: 4 workgroups drain ~500 items each replay, so
    # two replays started together overlap for most of their claims.
    monkeypatch.setenv("L20_PD_MAX_WORKGROUPS", "4")
    big = H.make_synthetic(8, 16, 2, 128, [4000, 3900, 4096, 3500, 4001, 3777, 4090, 3999], seed=31)
    tiny = H.make_synthetic(1, 16, 2, 128, [40], seed=32)
    split = 64
    outs = [torch.empty_like(big["query"]) for _ in range(2)]
    lses = [torch.empty(big["query"].shape[:2], dtype=torch.float32, device="cuda") for _ in range(2)]
    # every replay starts from zeroed outputs and partials, so an item that a
    # replay skipped cannot be covered by an earlier replay's partials
    wss = [H.workspace(big, split) for _ in range(2)]
    args_big = [cabi.args_from_tensors(big["query"], big["key_cache"], big["value_cache"], big["block_table"],
                                       big["seq_lens"], *wss[i], outs[i], big["k_scale"], big["v_scale"],
                                       big["max_seq_len"], split, softmax_scale=big["softmax_scale"], lse=lses[i])
                for i in range(2)]

    def zero(i):
        for t in (outs[i], lses[i]) + tuple(wss[i]):
            t.zero_()

    out_t = torch.empty_like(tiny["query"])
    lse_t = torch.empty(tiny["query"].shape[:2], dtype=torch.float32, device="cuda")
    args_tiny = _call_args(tiny, split, out_t, lse_t)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        cabi.split_out(args_big[0], stream.cuda_stream)
    torch.cuda.synchronize()
    ref = (outs[0].clone(), lses[0].clone())
    H.compare(*ref, *H.run_oracle(big))
    # 17 consecutive captures take the 16 capture slots in turn: the first and
    # the last share one.
    graphs = []
    for k in range(17):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                if k == 0:
                    cabi.split_out(args_big[0], stream.cuda_stream)
                elif k == 16:
                    cabi.split_out(args_big[1], stream.cuda_stream)
                else:
                    cabi.split_out(args_tiny, stream.cuda_stream)
        graphs.append(g)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    reported = exact = 0
    for rep in range(6):
        zero(0)
        zero(1)
        torch.cuda.synchronize()
        with torch.cuda.stream(sa):
            graphs[0].replay()
        with torch.cuda.stream(sb):
            graphs[16].replay()
        torch.cuda.synchronize()
        err = cabi.device_errors(clear=True)  # also zeroes the counters
        ok = all(torch.equal(outs[i], ref[0]) and torch.equal(lses[i], ref[1]) for i in range(2))
        assert err & ~cabi.L20_PD_DEVERR_QUEUE_SHARED == 0, err
        assert ok or err == cabi.L20_PD_DEVERR_QUEUE_SHARED, f"replay {rep}: wrong results and no report"
        reported += err != 0
        exact += ok
    print(f"overlapping replays on one slot: {reported} of 6 reported, {exact} of 6 exact", flush=True)
    # after the clear, the slot serves calls again
    for i, g in ((0, graphs[0]), (1, graphs[16])):
        zero(i)
        torch.cuda.synchronize()
        with torch.cuda.stream(sa):
            g.replay()
        torch.cuda.synchronize()
        assert cabi.device_errors() == 0
        assert torch.equal(outs[i], ref[0]) and torch.equal(lses[i], ref[1]), i


def test_graph_replay_soak_at_headline_scale():
    import l20_pd_cabi as cabi
    import l20_pd_workloads as wl

    cfg = wl.CONFIGS["c3_qwen2.5_7b"]
    inp = wl.make_inputs(cfg, device="cuda", seed=cfg.seed)
    split = cabi.load().l20_pd_default_split_size(cfg.batch, cfg.num_kv_heads, inp["max_seq_len"], 0)
    out = torch.empty_like(inp["query"])
    lse = torch.empty(inp["query"].shape[:2], dtype=torch.float32, device="cuda")
    args = _call_args(inp, split, out, lse)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        cabi.split_out(args, stream.cuda_stream)
    torch.cuda.synchronize()
    eager = (out.clone(), lse.clone())
    rows = [0, 1, 63, 64, 127]
    H.compare(*eager, *H.run_oracle(inp, rows=rows), rows=rows)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            cabi.split_out(args, stream.cuda_stream)
    torch.cuda.synchronize()
    mismatches = torch.zeros((), dtype=torch.int64, device="cuda")
    for i in range(1000):
        with torch.cuda.stream(stream):
            graph.replay()
            mismatches += (out != eager[0]).any().to(torch.int64) + (lse != eager[1]).any().to(torch.int64)
        if i % 100 == 99:
            torch.cuda.synchronize()
            assert int(mismatches) == 0, f"a replay before {i + 1} differs from the eager call"
    torch.cuda.synchronize()
    assert int(mismatches) == 0
    assert cabi.device_errors() == 0
