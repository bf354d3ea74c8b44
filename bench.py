#!/usr/bin/env python3
"""Benchmark of the MI355X paged FP8-KV decode-attention op.

One "step" is one decode-attention call (split-KV partial kernel + LSE merge
kernel) over one batch of the configured workload, with every input already
resident in HBM.  Steps rotate over several independently seeded input sets
whose K/V pools together exceed the 256 MB Infinity Cache, so each call reads
its KV cold from HBM.  Before the W warmup steps, untimed calls run for
``--settle-ms`` (250 ms) so that the timed loops start at steady GPU clocks
(reported as ``settle``).

Prints ONE JSON line (rank 0): value = KV-read GB/s of the whole call
(algorithmic K+V bytes / mean wall time per call, K back-to-back calls
between two events), plus the partial kernel's roofline (algorithmic KV
bytes / its own mean duration from HIP events recorded around it on the
launch stream, in a second timed loop: an event between the two kernels adds
a packet to the call) and a CPU baseline: a torch CPU restatement of the reference's
oracle timed on this host's usable cores over a bounded sample of the same
workload.

``--workload`` measures the other parts of the path the same way (the
default, ``decode``, is the headline):

* ``decode16`` -- the fp16/bf16-KV sibling (``paged_decode_split_out``) on the
  same shapes with bf16 caches;
* ``tree``     -- tree verification: the verify workload (config 5) with a
  random ancestor mask per sequence;
* ``kv_write`` -- the KV-cache producer (``rope_and_cache``): RoPE of Q and K
  and the paged fp8 write of K and V for a prefill chunk.
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
METRICS = {
    "decode": METRIC,
    "decode16": "KV-read HBM GB/s + µs per call, bf16-KV decode attention (paged_decode_split_out)",
    "tree": "KV-read HBM GB/s + µs per call, tree-verify attention (ancestor masks, q_len 4)",
    "kv_write": "HBM GB/s + µs per call, RoPE + paged fp8 KV write (rope_and_cache), prefill chunk",
}
DEFAULT_CONFIG = {"decode": "c3_qwen2.5_7b", "decode16": "c3_qwen2.5_7b", "tree": "c5_llama3_70b_verify",
                  "kv_write": "qwen2.5_7b_prefill16k"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=sorted(METRICS), default="decode")
    ap.add_argument("--config", default=None, help="workload configuration (default: the workload's own)")
    ap.add_argument("--split", type=int, default=0, help="split size (0 = library default)")
    ap.add_argument("--sets", type=int, default=0, help="rotating input sets (0 = enough to exceed 1 GB)")
    ap.add_argument("--hot", action="store_true", help="reuse one input set (cache-warm, informational)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--partial-dtype", choices=["fp32", "fp16"], default="fp16",
                    help="split-partial workspace dtype (the op accepts both; fp16 is the reference "
                         "op's own: half* partial_output, l20_paged_decode.cu:162,297)")
    ap.add_argument("--cpu-sample", type=int, default=0, help="sequences (tokens for kv_write) in the CPU sample")
    ap.add_argument("--settle-ms", type=float, default=250.0,
                    help="untimed calls before the warmup steps, until this much wall time has passed")
    ap.add_argument("--no-graph", dest="graph", action="store_false",
                    help="skip the informational HIP-graph replay of the timed calls (us_per_call_graph)")
    return ap.parse_args()


def settle(fn, min_ms: float, max_calls: int = 20000):
    """Untimed calls of ``fn(i)`` until ``min_ms`` of wall time have passed (at most
    ``max_calls``), so the timed loops start at steady GPU clocks: the first
    ~20 ms of back-to-back work in a process run measurably slower (config 3:
    55.3 instead of 53.8 us per call; config 5: 119 instead of 107).  Returns
    (calls made, milliseconds)."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while n < max_calls:
        for _ in range(16):
            fn(n)
            n += 1
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            break
    return n, (time.perf_counter() - t0) * 1e3


def cpu_threads():
    """Threads for the CPU baseline: the host CPUs this process may run on
    (``sched_getaffinity``), capped by ``OMP_NUM_THREADS`` when the host sets
    it (the GPU box gives one GPU's job a CPU share through it).  Returns
    ``(threads, cpus_visible)``."""
    visible = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(visible, int(omp)) if omp.isdigit() and int(omp) > 0 else visible
    return threads, visible


def sample_inputs(inp, rows):
    """The sequences ``rows`` of an input set, as numpy, with their pages
    renumbered into a compact pool (so the CPU side never copies the full cache)."""
    import numpy as np
    import torch

    bt = inp["block_table"].cpu().numpy()
    sl = inp["seq_lens"].cpu().numpy()
    q_len = inp["q_len"]
    pages, table = [], np.zeros((len(rows), bt.shape[1]), dtype=np.int32)
    for i, b in enumerate(rows):
        n = (int(sl[b]) + 15) // 16
        table[i, :n] = np.arange(len(pages), len(pages) + n)
        pages.extend(bt[b, :n].tolist())
    idx = torch.as_tensor(pages, dtype=torch.long, device=inp["key_cache"].device)

    def pick(c):
        sub = c.index_select(0, idx)
        return sub.view(torch.uint8).cpu().numpy() if c.dtype == torch.float8_e4m3fn else sub.float().cpu().numpy()

    q = inp["query"].float().cpu().numpy().reshape(-1, q_len, *inp["query"].shape[1:])[rows].reshape(
        -1, *inp["query"].shape[1:])
    tree = inp.get("tree_mask")
    tree = None if tree is None else tree.cpu().numpy().astype(np.int64)[rows]
    return q, pick(inp["key_cache"]), pick(inp["value_cache"]), table, sl[rows], tree


def host_scale(x):
    return x if isinstance(x, float) else x.float().cpu().numpy()


def oracle_call(inp, rows):
    """The CPU oracle over sequences ``rows``; returns ((out, lse), tokens, kv bytes, seconds)."""
    import torch
    from oracle import paged_fp8_decode_ref as ref

    q, kc, vc, bt, sl, tree = sample_inputs(inp, rows)
    t0 = time.perf_counter()
    if inp["key_cache"].dtype == torch.float8_e4m3fn:
        res = ref.reference(q, kc, vc, bt, sl, host_scale(inp["k_scale"]), host_scale(inp["v_scale"]),
                            softmax_scale=inp["softmax_scale"], q_len=inp["q_len"], tree_mask=tree)
    else:
        res = ref.reference_dense_kv(q, kc, vc, bt, sl, softmax_scale=inp["softmax_scale"], q_len=inp["q_len"],
                                     tree_mask=tree)
    return res, int(sl.sum()), kc.shape, time.perf_counter() - t0


def sample_inputs_torch(inp, rows):
    """CPU torch copies of the sequences ``rows`` of an input set (caches keep
    their dtype), pages renumbered into a compact pool."""
    import torch

    bt = inp["block_table"].cpu()
    sl = inp["seq_lens"].cpu()
    q_len = inp["q_len"]
    pages, table = [], torch.zeros((len(rows), bt.shape[1]), dtype=torch.int32)
    for i, b in enumerate(rows):
        n = (int(sl[b]) + 15) // 16
        table[i, :n] = torch.arange(len(pages), len(pages) + n, dtype=torch.int32)
        pages.extend(bt[b, :n].tolist())
    idx = torch.as_tensor(pages, dtype=torch.long, device=inp["key_cache"].device)
    q = inp["query"].cpu().view(-1, q_len, *inp["query"].shape[1:])[rows].reshape(-1, *inp["query"].shape[1:])
    tree = inp.get("tree_mask")

    def sc(x):
        return x if isinstance(x, float) else x.float().cpu()

    return {"query": q, "key_cache": inp["key_cache"].index_select(0, idx).cpu(),
            "value_cache": inp["value_cache"].index_select(0, idx).cpu(), "block_table": table,
            "seq_lens": sl[rows], "k_scale": sc(inp["k_scale"]), "v_scale": sc(inp["v_scale"]),
            "tree_mask": None if tree is None else tree.cpu()[rows]}


def cpu_baseline_decode(inp, cfg, sample_seqs, elem_bytes, min_seconds=10.0):
    """Time the torch CPU restatement of the reference's oracle over the first
    ``sample_seqs`` sequences of one input set, with one thread per usable host
    CPU: at least three calls, repeated until ``min_seconds`` of CPU work (at
    most 50 calls); the median call gives the rate."""
    import torch

    import l20_pd_workloads as wl
    from oracle import paged_fp8_decode_torch as tref

    threads, visible = cpu_threads()
    before = torch.get_num_threads()
    torch.set_num_threads(threads)
    s = sample_inputs_torch(inp, list(range(sample_seqs)))
    times = []
    try:
        while len(times) < 3 or (sum(times) < min_seconds and len(times) < 50):
            t0 = time.perf_counter()
            tref.reference_torch(s["query"], s["key_cache"], s["value_cache"], s["block_table"], s["seq_lens"],
                                 s["k_scale"], s["v_scale"], softmax_scale=inp["softmax_scale"], q_len=inp["q_len"],
                                 tree_mask=s["tree_mask"])
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(before)
    t = statistics.median(times)
    sl = s["seq_lens"]
    kv = wl.kv_bytes(sl, cfg.num_kv_heads, cfg.head_dim, elem_bytes)
    return {
        "value": round(kv / t / 1e9, 3),
        "unit": "GB/s",
        "cores": int(threads),
        "host_cpus_visible": int(visible),
        "kind": "port",
        "sample": f"torch CPU restatement of the reference's dequantise-then-attend oracle "
                  f"(scripts/smoke_cuda_paged_fp8_decode_op.py:22-41; oracle/paged_fp8_decode_torch.py, fp32, "
                  f"torch.set_num_threads({threads})) over sequences 0..{sample_seqs - 1} of the workload "
                  f"({int(sl.sum())} tokens, {kv / 1e6:.1f} MB KV), median of {len(times)} calls "
                  f"({sum(times):.1f} s of CPU work), {t * 1e3:.1f} ms per sample call",
        "us_per_call_sample": round(t * 1e6, 1),
    }


def measured_traffic(workload: str, split: int, kernel: str = "pd_fp8_partial", partial_dtype=None):
    """HBM bytes per launch of ``kernel`` from the committed counter profile
    (rocprofv3 FETCH_SIZE / WRITE_SIZE passes scaled by a copy of known size),
    or None when the profile has no entry for this workload, split and partial
    workspace dtype."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    for e in data["entries"]:
        if partial_dtype is not None and e.get("partial_dtype", "fp32") != partial_dtype:
            continue
        if e["workload"] == workload and e["split_size"] == split and e["kernel"] == kernel:
            read = e["fetch_kib"] * 1024 * data["fetch_scale"]
            write = e["write_kib"] * 1024 * data["write_scale"]
            return {"bytes": int(read + write), "read_bytes": int(read), "write_bytes": int(write),
                    "source": e.get("source", data["source"])}
    return None


def roofline(achieved, kernel, traffic, times_ms, mean_ms):
    """``achieved`` comes from ``mean_ms``: back-to-back launches of the kernel
    between two events.  ``times_ms`` are per-launch event intervals (each one
    also holds a dispatch and a completion signal), kept for the spread."""
    s = sorted(times_ms)
    return {
        "bound": "hbm",
        "kernel": kernel,
        "achieved": round(achieved, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic["bytes"] if traffic else None,
        "traffic_detail": traffic,
        "kernel_us_mean": round(mean_ms * 1e3, 2),
        "kernel_us_event_mean": round(statistics.mean(times_ms) * 1e3, 2),
        "kernel_us_event_p10_p90": [round(s[len(s) // 10] * 1e3, 2), round(s[(9 * len(s)) // 10] * 1e3, 2)],
    }


def random_tree_words(batch, q_len, seed):
    """int32 [batch, q_len] ancestor words of random draft trees (parent index < child)."""
    import numpy as np
    import torch

    rng = np.random.default_rng(seed)
    words = np.zeros((batch, q_len), dtype=np.int64)
    for b in range(batch):
        parent = [-1] + [int(rng.integers(-1, i)) for i in range(1, q_len)]
        for i in range(q_len):
            j = i
            while j >= 0:
                words[b, i] |= 1 << j
                j = parent[j]
    return torch.from_numpy(np.where(words >= 2**31, words - 2**32, words).astype(np.int32))


def run_decode(args, mode):
    """decode / decode16 / tree: partial + merge per step through the C ABI."""
    import torch

    import l20_pd_cabi as cabi
    import l20_pd_workloads as wl
    import l20_paged_decode  # noqa: F401  (fails loudly without the extension)

    dev = torch.device("cuda:0")
    cfg = wl.CONFIGS[args.config or DEFAULT_CONFIG[mode]]
    lib = cabi.load()
    props = torch.cuda.get_device_properties(dev)
    kv_dtype = torch.bfloat16 if mode == "decode16" else None
    elem = 2 if kv_dtype is not None else 1

    def make(seed):
        inp = wl.make_inputs(cfg, device=dev, seed=seed, kv_dtype=kv_dtype)
        if mode == "tree":
            inp["tree_mask"] = random_tree_words(cfg.batch, cfg.q_len, seed).to(dev)
        return inp

    first = make(cfg.seed)
    pool_bytes = 2 * first["key_cache"].numel() * first["key_cache"].element_size()
    # enough sets to exceed 1 GB (at most 64: the tiny configs are launch-bound anyway)
    n_sets = 1 if args.hot else (args.sets or min(64, max(3, -(-1_000_000_000 // pool_bytes))))
    sets = [first] + [make(cfg.seed + 1000 * i) for i in range(1, n_sets)]
    max_seq = max(s["max_seq_len"] for s in sets)
    split = args.split or int(lib.l20_pd_default_split_size(cfg.batch, cfg.num_kv_heads, max_seq,
                                                            props.multi_processor_count))
    n_s = max(1, -(-max_seq // split))
    rows = cfg.batch * cfg.q_len
    stream = torch.cuda.current_stream(dev)

    calls = []
    for s in sets:
        po = torch.empty(rows, cfg.num_q_heads, n_s, cfg.head_dim,
                         dtype=torch.float16 if args.partial_dtype == "fp16" else torch.float32, device=dev)
        pm = torch.empty(rows, cfg.num_q_heads, n_s, dtype=torch.float32, device=dev)
        ps = torch.empty_like(pm)
        out = torch.empty_like(s["query"])
        lse = torch.empty(rows, cfg.num_q_heads, dtype=torch.float32, device=dev)
        ks, ksph = (s["k_scale"], None) if isinstance(s["k_scale"], float) else (1.0, s["k_scale"])
        vs, vsph = (s["v_scale"], None) if isinstance(s["v_scale"], float) else (1.0, s["v_scale"])
        a = cabi.args_from_tensors(s["query"], s["key_cache"], s["value_cache"], s["block_table"], s["seq_lens"],
                                   po, pm, ps, out, ks, vs, s["max_seq_len"], split, softmax_scale=s["softmax_scale"],
                                   k_scale_per_head=ksph, v_scale_per_head=vsph, q_len=cfg.q_len, lse=lse,
                                   tree_mask=s.get("tree_mask"))
        calls.append((a, (po, pm, ps, out, lse)))
    kvb = [wl.kv_bytes(s["seq_lens"], cfg.num_kv_heads, cfg.head_dim, elem) for s in sets]
    h = stream.cuda_stream
    # Small batches of short sequences run as one launch (pd_fp8_fused, no
    # merge): that kernel is then the call, and the roofline times it as such.
    # Batches whose 512-token splits fill the CUs once run the partial stage
    # as that kernel's split mode (then the merge): the roofline times it.
    path = cabi.launch_path(calls[0][0], lib)
    single = path == 1
    kernel = "pd_fp8_fused" if path else "pd_fp8_partial"
    kernel_fn = cabi.split_out if single else cabi.partial

    settle_calls, settle_ms = settle(lambda i: cabi.split_out(calls[i % n_sets][0], h, lib), args.settle_ms)
    for i in range(args.warmup):
        cabi.split_out(calls[i % n_sets][0], h, lib)
    torch.cuda.synchronize()

    # Timed region 1 (value): K whole calls (partial + merge, as the op
    # enqueues them), bracketed by events only -- an event between the two
    # kernels would add its own packet to every call.
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for k in range(args.steps):
        cabi.split_out(calls[k % n_sets][0], h, lib)
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / args.steps
    # Timed region 2 (roofline): K partial launches back to back on the launch
    # stream between two events (the merge is not needed to time the partial
    # kernel; every launch rewrites the same workspace), or K single launches.
    p_start, p_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    p_start.record(stream)
    for k in range(args.steps):
        kernel_fn(calls[k % n_sets][0], h, lib)
    p_end.record(stream)
    torch.cuda.synchronize()
    partial_mean_ms = p_start.elapsed_time(p_end) / args.steps
    # Region 3 (spread only): events around every partial launch of whole calls.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for k in range(args.steps):
        a = calls[k % n_sets][0]
        ev[k][0].record(stream)
        kernel_fn(a, h, lib)
        ev[k][1].record(stream)
        if not single:
            cabi.merge(a, h, lib)
    torch.cuda.synchronize()
    partial_ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    # Region 4 (informational): the same K calls captured once into a HIP graph
    # and replayed, which takes the host's per-launch cost (~2 us of ctypes and
    # hipLaunchKernel per kernel) out of the small configurations' times.
    graph_ms = None
    if args.graph:
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for k in range(args.steps):
                    cabi.split_out(calls[k % n_sets][0], side.cuda_stream, lib)
        torch.cuda.synchronize()
        # The capture leaves the GPU idle long enough for its clocks to drop
        # (a call right after 2 s of idling: config 4 95.1 instead of 90.0 us),
        # so the replays settle like the eager loops before three are timed.
        with torch.cuda.stream(side):
            settle(lambda i: graph.replay(), args.settle_ms, max_calls=16 * max(1, -(-2000 // args.steps)))
            g_start, g_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            g_start.record(side)
            for _ in range(3):
                graph.replay()
            g_end.record(side)
        torch.cuda.synchronize()
        graph_ms = g_start.elapsed_time(g_end) / (3 * args.steps)
        del graph
    bytes_per_step = sum(kvb[k % n_sets] for k in range(args.steps)) / args.steps
    value = bytes_per_step / (ms_per_step * 1e-3) / 1e9
    achieved = bytes_per_step / (partial_mean_ms * 1e-3) / 1e9

    check = None
    if not args.no_check:
        import numpy as np
        import pd_helpers as H

        a, (po, pm, ps, out, lse) = calls[0]
        cabi.split_out(a, h, lib)
        torch.cuda.synchronize()
        sample = list(range(min(8 if mode != "tree" else 3, cfg.batch)))
        (exp_out, exp_lse), _, _, _ = oracle_call(first, sample)
        r = np.concatenate([np.arange(b * cfg.q_len, (b + 1) * cfg.q_len) for b in sample])
        full_out = np.zeros((rows,) + exp_out.shape[1:], dtype=np.float32)
        full_lse = np.zeros((rows,) + exp_lse.shape[1:], dtype=np.float32)
        full_out[r], full_lse[r] = exp_out, exp_lse
        check = H.compare(out, lse, full_out, full_lse, rows=r)

    cpu = None
    if not args.no_cpu_baseline:
        sample = args.cpu_sample or (cfg.batch if mode == "decode" else min(cfg.batch, 4))
        cpu = cpu_baseline_decode(first, cfg, sample, elem)

    workload = cfg.name + {"decode": "", "decode16": "+bf16kv", "tree": "+tree"}[mode]
    traffic = measured_traffic(workload, split, kernel=kernel, partial_dtype=None if single else args.partial_dtype)
    line = {
        "metric": METRICS[mode],
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"calls": settle_calls, "ms": round(settle_ms, 1)},
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 2),
        "us_per_call_graph": None if graph_ms is None else round(graph_ms * 1e3, 2),
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16 KV x bf16 Q -> f32 accumulate (bf16 MFMA, P split hi+lo)" if mode == "decode16" else
                  "fp8e4m3 KV x bf16 Q -> f32 accumulate (bf16/f16 MFMA)"),
        "data": ("synthetic (seeded N(0,1) bf16 query, N(0,1) bf16 keys/values)" if mode == "decode16" else
                 "synthetic (seeded N(0,1) bf16 query, N(0,1) keys/values quantised to e4m3fn)"
                 + (", random draft trees" if mode == "tree" else "")),
        "config": {
            "workload": workload,
            "batch": cfg.batch, "q_heads": cfg.num_q_heads, "kv_heads": cfg.num_kv_heads,
            "head_dim": cfg.head_dim, "q_len": cfg.q_len, "page_size": 16,
            "seq_lens": (f"lognormal(median {cfg.lognormal_median}, sigma {wl.LOGNORMAL_SIGMA}) clipped "
                         f"{list(cfg.lognormal_clip)}" if cfg.lognormal_median else
                         (f"fixed {cfg.context}" if cfg.context else f"uniform {list(cfg.seq_len_range)}")),
            "scales": "none (16-bit KV)" if mode == "decode16" else (
                "per-head" if cfg.per_head_scales else "per-tensor"),
            "mask": "tree (random ancestor words per sequence)" if mode == "tree" else (
                "causal over the q_len new tokens" if cfg.q_len > 1 else "none"),
            "split_size": split,
            "partial_dtype": args.partial_dtype,
            "kv_bytes_per_call": int(bytes_per_step),
            "input_sets": n_sets,
            "cache_state": "hot (one set)" if args.hot else (
                f"{'cold' if n_sets * pool_bytes > 512e6 else 'Infinity-Cache resident'}: {n_sets} rotating sets, "
                f"{n_sets * pool_bytes / 1e6:.0f} MB of K/V pools"),
            "parallelism": "single GPU",
        },
        "roofline": roofline(achieved, kernel, traffic, partial_ms, partial_mean_ms),
        "cpu_baseline": cpu,
        "parity": check,
        "device": getattr(props, "gcnArchName", props.name),
    }
    # the headline line keeps its established field name for the kernel's mean time
    line["roofline"]["partial_us_mean"] = line["roofline"]["kernel_us_mean"]
    line["roofline"]["partial_us_event_p10_p90"] = line["roofline"]["kernel_us_event_p10_p90"]
    return line


# --------------------------------------------------------------------------- kv_write
KV_WRITE = {"qwen2.5_7b_prefill16k": dict(tokens=16384, q_heads=28, kv_heads=4, head_dim=128, rotary_dim=128,
                                          max_position=32768, is_neox=True, seed=53)}


def kv_write_bytes(c):
    """Algorithmic HBM bytes of one call: read Q, K, V (bf16), the token's cos/sin
    row (bf16), position and slot (int64); write Q, K back and the fp8 K, V rows."""
    t, d = c["tokens"], c["head_dim"]
    q, kv = t * c["q_heads"] * d * 2, t * c["kv_heads"] * d * 2
    read = q + 2 * kv + t * c["rotary_dim"] * 2 + 2 * t * 8
    write = q + kv + 2 * t * c["kv_heads"] * d
    return read + write


def run_kv_write(args):
    import numpy as np
    import torch

    import l20_rope_kv

    dev = torch.device("cuda:0")
    name = args.config or DEFAULT_CONFIG["kv_write"]
    c = KV_WRITE[name]
    props = torch.cuda.get_device_properties(dev)
    T, hq, hkv, d = c["tokens"], c["q_heads"], c["kv_heads"], c["head_dim"]

    def make(seed):
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(T, hq, d, generator=g).to(torch.bfloat16).to(dev)
        k = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        start = int(torch.randint(0, c["max_position"] - T, (1,), generator=g))
        pos = torch.arange(start, start + T, dtype=torch.int64).to(dev)
        pages = (T + 15) // 16
        pool = pages + pages // 4
        perm = torch.randperm(pool, generator=g)[:pages]
        t = torch.arange(T)
        slots = (perm[t // 16] * 16 + t % 16).to(torch.int64).to(dev)
        kc = torch.zeros(pool, 16, hkv, d, dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.zeros_like(kc)
        return {"q": q, "k": k, "v": v, "pos": pos, "slots": slots, "kc": kc, "vc": vc}

    gcs = torch.Generator().manual_seed(c["seed"])
    theta = torch.rand(c["max_position"], c["rotary_dim"] // 2, generator=gcs, dtype=torch.float64) * 6.2831853
    cos_sin = torch.cat([theta.cos(), theta.sin()], -1).to(torch.bfloat16).to(dev)
    first = make(c["seed"])
    per_set = sum(x.numel() * x.element_size() for x in first.values())
    n_sets = 1 if args.hot else (args.sets or max(3, -(-1_000_000_000 // per_set)))
    sets = [first] + [make(c["seed"] + 1000 * i) for i in range(1, n_sets)]
    # per-head scales of the first set's values (the producer's own scale kernel)
    ks, vs = l20_rope_kv.l20_kv_fp8_scales(first["k"], first["v"], first["pos"], cos_sin, c["is_neox"],
                                           first["kc"], first["vc"], first["slots"])

    def call(s):
        l20_rope_kv.l20_rope_and_cache(s["q"], s["k"], s["v"], s["pos"], cos_sin, c["is_neox"], s["kc"], s["vc"],
                                       s["slots"], k_scale_per_head=ks, v_scale_per_head=vs)

    # keep pristine copies of the first set for the parity check (calls rotate Q and K in place)
    q0, k0 = first["q"].clone(), first["k"].clone()
    settle_calls, settle_ms = settle(lambda i: call(sets[i % n_sets]), args.settle_ms)
    for i in range(args.warmup):
        call(sets[i % n_sets])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    # value and roofline: K back-to-back calls between two events (a call with
    # given scales is one launch of the producer kernel); a second loop with
    # events around every call gives the spread
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start.record(stream)
    for k in range(args.steps):
        call(sets[k % n_sets])
    t_end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t_start.elapsed_time(t_end) / args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for k in range(args.steps):
        ev[k][0].record(stream)
        call(sets[k % n_sets])
        ev[k][1].record(stream)
    torch.cuda.synchronize()
    kern_ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    nbytes = kv_write_bytes(c)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    achieved = value

    from oracle import kv_write_ref as kref

    def oracle_sample(n):
        cs_np = cos_sin.float().cpu().numpy()
        pos = first["pos"][:n].cpu().numpy()
        slots_local = np.arange(n)  # a compact pool for the sample
        pages = (n + 15) // 16
        kc = np.zeros((pages, 16, hkv, d), dtype=np.uint8)
        t0 = time.perf_counter()
        res = kref.rope_and_cache(q0[:n].float().cpu().numpy(), k0[:n].float().cpu().numpy(),
                                  first["v"][:n].float().cpu().numpy(), pos, cs_np, c["is_neox"], kc, kc.copy(),
                                  slots_local, dtype="bf16", cache_fp8=True, k_scale=ks.cpu().numpy(),
                                  v_scale=vs.cpu().numpy())
        return res, time.perf_counter() - t0

    check = None
    if not args.no_check:
        n = 1024
        s = dict(first, q=q0[:n].clone(), k=k0[:n].clone(), v=first["v"][:n], pos=first["pos"][:n],
                 slots=torch.arange(n, dtype=torch.int64, device=dev),
                 kc=torch.zeros((n + 15) // 16, 16, hkv, d, dtype=torch.float8_e4m3fn, device=dev))
        s["vc"] = torch.zeros_like(s["kc"])
        call(s)
        torch.cuda.synchronize()
        (q_e, k_e, kc_e, vc_e), _ = oracle_sample(n)
        got = [s["q"].float().cpu().numpy(), s["k"].float().cpu().numpy(),
               s["kc"].view(torch.uint8).cpu().numpy(), s["vc"].view(torch.uint8).cpu().numpy()]
        exact = [bool(np.array_equal(a, b)) for a, b in zip(got, [q_e, k_e, kc_e, vc_e])]
        check = {"tokens": n, "bit_exact_q_k_kcache_vcache": exact}
        assert all(exact), check

    cpu = None
    if not args.no_cpu_baseline:
        n = args.cpu_sample or 4096
        times = []  # at least three calls, up to ~10 s of CPU work (at most 50 calls)
        while len(times) < 3 or (sum(times) < 10.0 and len(times) < 50):
            times.append(oracle_sample(n)[1])
        t = statistics.median(times)
        sample_bytes = kv_write_bytes(dict(c, tokens=n))
        cpu = {"value": round(sample_bytes / t / 1e9, 4), "unit": "GB/s", "cores": 1,
               "host_cpus_visible": int(cpu_threads()[1]), "kind": "port",
               "sample": f"numpy oracle (oracle/kv_write_ref.py; elementwise numpy, one thread) over the first "
                         f"{n} tokens of the chunk "
                         f"({sample_bytes / 1e6:.1f} MB of algorithmic traffic), median of {len(times)} calls "
                         f"({sum(times):.1f} s of CPU work), {t * 1e3:.1f} ms per sample call"}

    return {
        "metric": METRICS["kv_write"],
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"calls": settle_calls, "ms": round(settle_ms, 1)},
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 2),
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 Q/K/V -> f32 RoPE (no contraction) -> bf16 Q/K; fp8e4m3 K/V cache (RNE, per-head scales)",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, random rotary angles, consecutive positions, random pages)",
        "config": {"workload": "kv_write_" + name, **{k: v for k, v in c.items() if k != "seed"},
                   "cache": "fp8 e4m3fn [pages, 16, Hkv, D]", "scales": "per-head",
                   "bytes_per_call": nbytes, "input_sets": n_sets, "parallelism": "single GPU"},
        "roofline": roofline(achieved, "kv_rope_write", measured_traffic("kv_write_" + name, 0, "kv_rope_write"),
                             kern_ms, ms_per_step),
        "cpu_baseline": cpu,
        "parity": check,
        "device": getattr(props, "gcnArchName", props.name),
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: decode attention on one GPU's "
                                   "share needs no collectives; --gpus above 1 is not supported"}))
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    torch.cuda.set_device(torch.device("cuda:0"))
    line = run_kv_write(args) if args.workload == "kv_write" else run_decode(args, args.workload)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
