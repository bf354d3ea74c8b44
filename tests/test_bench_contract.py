"""bench.py's output contract: one JSON line with the fields the driver reads.

The CPU test checks the one-GPU refusal; the GPU test runs a short headline
bench in a child process (its own GPU context, a time limit) and checks every
field of the line.
"""

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args, timeout=240):
    return subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run_bench("--gpus", "2", timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "exactly one GPU" in line["error"]


@pytest.mark.gpu
def test_headline_line_carries_every_contract_field():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    r = run_bench("--steps", "10", "--warmup", "3", "--no-cpu-baseline")
    assert r.returncode == 0, r.stderr[-2000:]
    d = json.loads(r.stdout.strip().splitlines()[-1])
    assert d["metric"].startswith("KV-read HBM GB/s") and d["unit"] == "GB/s"
    assert d["value"] > 0 and d["ms_per_step"] > 0
    assert d["n_gpus"] == 1 and d["steps"] == 10 and d["warmup"] == 3
    assert d["higher_is_better"] is True and d["scaling"] in ("weak", "strong")
    assert d["vs_baseline"] is None
    assert d["dtype"].startswith("fp8e4m3") and d["data"].startswith("synthetic")
    assert d["config"]["workload"] == "c3_qwen2.5_7b"
    # value is KV bytes over the mean call time
    assert abs(d["value"] - d["config"]["kv_bytes_per_call"] / (d["ms_per_step"] * 1e-3) / 1e9) < 0.01 * d["value"]
    r0 = d["roofline"]
    assert r0["bound"] == "hbm" and r0["unit"] == "GB/s" and r0["peak"] == 8000.0
    assert 0 < r0["achieved"] and abs(r0["frac"] - r0["achieved"] / r0["peak"]) < 1e-3
    assert r0["traffic"] is None or r0["traffic"] > d["config"]["kv_bytes_per_call"]
    assert d["cpu_baseline"] is None  # disabled by the flag
    assert d["parity"]["min_cos"] >= 0.9999


def test_cpu_baseline_fields_on_the_cpu(monkeypatch):
    """The CPU baseline times the torch restatement with one thread per usable
    host CPU (capped by OMP_NUM_THREADS) and reports that count as ``cores``."""
    import os
    import types

    import pd_helpers as H

    sys.path.insert(0, str(ROOT))
    import bench

    monkeypatch.setenv("OMP_NUM_THREADS", "2")
    inp = H.make_synthetic(3, 8, 2, 64, [40, 17, 90], seed=4, device="cpu")
    cfg = types.SimpleNamespace(num_kv_heads=2, head_dim=64)
    cpu = bench.cpu_baseline_decode(inp, cfg, 2, 1, min_seconds=0.01)
    assert cpu["kind"] == "port" and cpu["unit"] == "GB/s" and cpu["value"] > 0
    assert cpu["cores"] == min(2, len(os.sched_getaffinity(0)))
    assert cpu["host_cpus_visible"] == len(os.sched_getaffinity(0))
    assert "torch CPU restatement" in cpu["sample"] and "57 tokens" in cpu["sample"]
