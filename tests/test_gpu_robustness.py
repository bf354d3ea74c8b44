"""Robustness of the persistent partial kernel (GPU).

* Bounded hand-off waits: with a spin limit of one poll (set from the host
  with l20_pd_set_spin_limit) the waits between the waves of a workgroup give
  up at once; every kernel still exits normally, the give-up is reported through
  l20_pd_device_errors, and after clearing it the next call is exact again.
* Counter slots: graph replays of a queue-driven call interleaved with eager
  queue-driven calls on another stream, each bitwise equal to its eager
  result (a graph's captured launch and the other stream's launches hold
  different work-queue slots).
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
    assert err != 0 and err & ~7 == 0, err
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
