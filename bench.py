#!/usr/bin/env python3
"""Benchmark of the MI355X paged FP8-KV decode-attention op.

One "step" is one decode-attention call (split-KV partial kernel + LSE merge
kernel) over one batch of the configured workload, with every input already
resident in HBM.  Steps rotate over several independently seeded input sets
whose K/V pools together exceed the 256 MB Infinity Cache, so each call reads
its KV cold from HBM.

Prints ONE JSON line (rank 0): value = KV-read GB/s of the whole call
(algorithmic K+V bytes / mean wall time per call), plus the partial kernel's
roofline (algorithmic KV bytes / its own mean duration from HIP events
recorded around it on the launch stream) and a CPU baseline: the CPU oracle
timed on this host over a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "single-gpu-inference-lab_amd"), str(ROOT), str(ROOT / "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "KV-read HBM GB/s (% of ~8 TB/s) + µs per decode-attn call, 7B-shape batch 128"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3_qwen2.5_7b")
    ap.add_argument("--split", type=int, default=0, help="split size (0 = library default)")
    ap.add_argument("--sets", type=int, default=0, help="rotating input sets (0 = enough to exceed 1 GB)")
    ap.add_argument("--hot", action="store_true", help="reuse one input set (cache-warm, informational)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=0, help="sequences in the CPU-baseline sample (0 = auto)")
    return ap.parse_args()


def cpu_baseline(inp, cfg, sample_seqs):
    """Time the CPU oracle over the first ``sample_seqs`` sequences of one input set."""
    import numpy as np
    import torch
    from oracle import paged_fp8_decode_ref as ref

    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover - threadpoolctl is optional
        threads = 1
    q = inp["query"].float().cpu().numpy()
    kc = inp["key_cache"].view(torch.uint8).cpu().numpy()
    vc = inp["value_cache"].view(torch.uint8).cpu().numpy()
    bt = inp["block_table"].cpu().numpy()
    sl = inp["seq_lens"].cpu().numpy()
    ks = inp["k_scale"] if isinstance(inp["k_scale"], float) else inp["k_scale"].cpu().numpy()
    vs = inp["v_scale"] if isinstance(inp["v_scale"], float) else inp["v_scale"].cpu().numpy()
    rows = list(range(sample_seqs))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        ref.reference(q, kc, vc, bt, sl, ks, vs, softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], rows=rows)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    kv = ref.kv_bytes(sl[:sample_seqs], cfg.num_kv_heads, cfg.head_dim)
    return {
        "value": round(kv / t / 1e9, 3),
        "unit": "GB/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"numpy oracle (oracle/paged_fp8_decode_ref.py) over sequences 0..{sample_seqs - 1} of the "
                  f"workload ({int(sl[:sample_seqs].sum())} tokens, {kv / 1e6:.1f} MB KV), median of 3, "
                  f"{t * 1e3:.1f} ms per sample call",
        "us_per_call_sample": round(t * 1e6, 1),
    }


def measured_traffic(workload: str, split: int, kernel: str = "pd_fp8_partial"):
    """HBM bytes per launch of ``kernel`` from the committed counter profile
    (rocprofv3 FETCH_SIZE / WRITE_SIZE passes scaled by a copy of known size),
    or None when the profile has no entry for this workload and split."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    for e in data["entries"]:
        if e["workload"] == workload and e["split_size"] == split and e["kernel"] == kernel:
            read = e["fetch_kib"] * 1024 * data["fetch_scale"]
            write = e["write_kib"] * 1024 * data["write_scale"]
            return {"bytes": int(read + write), "read_bytes": int(read), "write_bytes": int(write),
                    "source": data["source"]}
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: decode attention on one GPU's "
                                   "share needs no collectives; --gpus above 1 is not supported"}))
        sys.exit(2)

    import torch

    import l20_pd_cabi as cabi
    import l20_pd_workloads as wl
    import l20_paged_decode  # noqa: F401  (fails loudly without the extension)

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = wl.CONFIGS[args.config]
    lib = cabi.load()
    props = torch.cuda.get_device_properties(dev)

    first = wl.make_inputs(cfg, device=dev)
    kv_bytes = wl.kv_bytes(first["seq_lens"], cfg.num_kv_heads, cfg.head_dim)
    pool_bytes = 2 * first["key_cache"].numel()
    n_sets = 1 if args.hot else (args.sets or max(3, -(-1_000_000_000 // pool_bytes)))
    sets = [first] + [wl.make_inputs(cfg, device=dev, seed=cfg.seed + 1000 * i) for i in range(1, n_sets)]
    max_seq = max(s["max_seq_len"] for s in sets)
    split = args.split or int(lib.l20_pd_default_split_size(cfg.batch, cfg.num_kv_heads, max_seq,
                                                            props.multi_processor_count))
    n_s = max(1, -(-max_seq // split))
    rows = cfg.batch * cfg.q_len
    stream = torch.cuda.current_stream(dev)

    calls = []
    for s in sets:
        po = torch.empty(rows, cfg.num_q_heads, n_s, cfg.head_dim, dtype=torch.float32, device=dev)
        pm = torch.empty(rows, cfg.num_q_heads, n_s, dtype=torch.float32, device=dev)
        ps = torch.empty_like(pm)
        out = torch.empty_like(s["query"])
        lse = torch.empty(rows, cfg.num_q_heads, dtype=torch.float32, device=dev)
        ks, ksph = (s["k_scale"], None) if isinstance(s["k_scale"], float) else (1.0, s["k_scale"])
        vs, vsph = (s["v_scale"], None) if isinstance(s["v_scale"], float) else (1.0, s["v_scale"])
        a = cabi.args_from_tensors(s["query"], s["key_cache"], s["value_cache"], s["block_table"], s["seq_lens"],
                                   po, pm, ps, out, ks, vs, max_seq, split, softmax_scale=s["softmax_scale"],
                                   k_scale_per_head=ksph, v_scale_per_head=vsph, q_len=cfg.q_len, lse=lse)
        calls.append((a, (po, pm, ps, out, lse)))
    kvb = [wl.kv_bytes(s["seq_lens"], cfg.num_kv_heads, cfg.head_dim) for s in sets]
    h = stream.cuda_stream

    for i in range(args.warmup):
        cabi.split_out(calls[i % n_sets][0], h, lib)
    torch.cuda.synchronize()

    # Timed region: K calls; events around every partial launch on the same stream.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for k in range(args.steps):
        a = calls[k % n_sets][0]
        ev[k][0].record(stream)
        cabi.partial(a, h, lib)
        ev[k][1].record(stream)
        cabi.merge(a, h, lib)
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / args.steps
    partial_ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    bytes_per_step = sum(kvb[k % n_sets] for k in range(args.steps)) / args.steps
    partial_mean_ms = statistics.mean(partial_ms)
    value = bytes_per_step / (ms_per_step * 1e-3) / 1e9
    achieved = bytes_per_step / (partial_mean_ms * 1e-3) / 1e9

    check = None
    if not args.no_check:
        import numpy as np
        import pd_helpers as H

        a, (po, pm, ps, out, lse) = calls[0]
        cabi.split_out(a, h, lib)
        torch.cuda.synchronize()
        sample = list(range(min(8, cfg.batch)))
        exp_out, exp_lse = H.run_oracle(first, rows=sample)
        r = np.concatenate([np.arange(b * cfg.q_len, (b + 1) * cfg.q_len) for b in sample])
        check = H.compare(out, lse, exp_out, exp_lse, rows=r)

    cpu = None
    if not args.no_cpu_baseline:
        sample = args.cpu_sample or min(cfg.batch, 32)
        cpu = cpu_baseline(first, cfg, sample)

    traffic = measured_traffic(cfg.name, split)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 2),
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 KV x bf16 Q -> f32 accumulate (bf16/f16 MFMA)",
        "data": "synthetic (seeded N(0,1) bf16 query, N(0,1) keys/values quantised to e4m3fn)",
        "config": {
            "workload": cfg.name,
            "batch": cfg.batch, "q_heads": cfg.num_q_heads, "kv_heads": cfg.num_kv_heads,
            "head_dim": cfg.head_dim, "q_len": cfg.q_len, "page_size": 16,
            "seq_lens": (f"lognormal(median {cfg.lognormal_median}, sigma {wl.LOGNORMAL_SIGMA}) clipped "
                         f"{list(cfg.lognormal_clip)}" if cfg.lognormal_median else
                         (f"fixed {cfg.context}" if cfg.context else f"uniform {list(cfg.seq_len_range)}")),
            "scales": "per-head" if cfg.per_head_scales else "per-tensor",
            "split_size": split,
            "kv_bytes_per_call": int(bytes_per_step),
            "input_sets": n_sets,
            "cache_state": "hot (one set)" if args.hot else f"cold: {n_sets} rotating sets, "
                                                           f"{n_sets * pool_bytes / 1e6:.0f} MB of K/V pools",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "pd_fp8_partial",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_detail": traffic,
            "partial_us_mean": round(partial_mean_ms * 1e3, 2),
            "partial_us_p10_p90": [round(sorted(partial_ms)[len(partial_ms) // 10] * 1e3, 2),
                                   round(sorted(partial_ms)[(9 * len(partial_ms)) // 10] * 1e3, 2)],
        },
        "cpu_baseline": cpu,
        "parity": check,
        "device": getattr(props, "gcnArchName", props.name),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
