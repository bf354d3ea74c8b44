"""GPU: the patched stand-in vLLM forward dispatches decode to the MI355X op."""

import importlib
import json
import shutil
import sys
import types
from pathlib import Path

import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu
FIXTURE = Path(__file__).parent / "fixtures" / "vllm_rocm"


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")


def test_patched_forward_runs_the_op_and_traces(tmp_path, monkeypatch):
    import install_l20_fp8_paged_decode_rocm as inst
    import l20_vllm_rocm_hook as hook

    shutil.copytree(FIXTURE, tmp_path / "src")
    inst.main(["--vllm-source-dir", str(tmp_path / "src")])
    monkeypatch.syspath_prepend(str(tmp_path / "src"))
    for name in [m for m in sys.modules if m == "vllm" or m.startswith("vllm.")]:
        monkeypatch.delitem(sys.modules, name)
    mod = importlib.import_module("vllm.v1.attention.backends.triton_attn")
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv(hook.ENABLE_ENV, "1")
    monkeypatch.setenv(hook.TRACE_ENV, str(trace))
    # the heuristic gate is closed, as in the reference: FORCE opens the path
    monkeypatch.setenv(hook.FORCE_ENV, "1")

    inp = H.make_synthetic(6, 16, 2, 128, [700, 31, 2048, 1, 300, 999], seed=12)
    kv = torch.stack([inp["key_cache"].view(torch.uint8), inp["value_cache"].view(torch.uint8)])  # [2, P, 16, Hkv, D]
    impl = mod.TritonAttentionImpl(16, 128, inp["softmax_scale"], 2, kv_cache_dtype="fp8_e4m3")
    layer = types.SimpleNamespace(_k_scale_float=inp["k_scale"], _v_scale_float=inp["v_scale"])
    meta = types.SimpleNamespace(num_actual_tokens=6, query_start_loc=None, seq_lens=inp["seq_lens"],
                                 max_query_len=1, max_seq_len=inp["max_seq_len"], block_table=inp["block_table"])
    out = torch.full((8, 16, 128), 7.0, dtype=torch.bfloat16, device="cuda")  # padded token rows stay untouched
    q = torch.cat([inp["query"], torch.zeros(2, 16, 128, dtype=torch.bfloat16, device="cuda")])
    for _ in range(2):  # the second call reuses the cached workspace
        impl.forward(layer, q, None, None, kv, meta, output=out)
    torch.cuda.synchronize()
    assert mod.CALLS == []  # vLLM's kernel did not run
    exp_out, _ = H.run_oracle(inp)
    H.compare(out[:6], None, exp_out, None, check_lse=False)
    assert bool((out[6:] == 7.0).all())
    lines = [json.loads(x) for x in trace.read_text().splitlines()]
    assert len(lines) == 2 and lines[0] == {"event": "l20_fp8_paged_decode_run", "batch": 6,
                                            "max_seq_len": 2048, "q_heads": 16, "kv_heads": 2}
    # a prefill batch falls back to vLLM's kernel
    meta.max_query_len = 4
    impl.forward(layer, q, None, None, kv, meta, output=out)
    assert len(mod.CALLS) == 1
    # so do a decode batch without FORCE (closed heuristic gate), a fused
    # output quantisation and an fp8 output buffer
    meta.max_query_len = 1
    monkeypatch.delenv(hook.FORCE_ENV)
    impl.forward(layer, q, None, None, kv, meta, output=out)
    assert len(mod.CALLS) == 2
    monkeypatch.setenv(hook.FORCE_ENV, "1")
    impl.forward(layer, q, None, None, kv, meta, output=out, output_scale=torch.ones((), device="cuda"))
    assert len(mod.CALLS) == 3
    impl.forward(layer, q, None, None, kv, meta, output=torch.zeros(8, 16, 128, device="cuda").to(torch.float8_e4m3fn))
    assert len(mod.CALLS) == 4
    assert len(trace.read_text().splitlines()) == 2


def test_patched_forward_reads_e5m2_caches_in_their_format(tmp_path, monkeypatch):
    """kv_cache_dtype "fp8_e5m2": vLLM's backend views the cache as its platform
    fp8 type (e4m3fn here); the hook re-views the bytes as e5m2, so the result
    is the e5m2 oracle's, not that of the same bytes read as e4m3fn."""
    import install_l20_fp8_paged_decode_rocm as inst
    import l20_vllm_rocm_hook as hook

    shutil.copytree(FIXTURE, tmp_path / "src")
    inst.main(["--vllm-source-dir", str(tmp_path / "src")])
    monkeypatch.syspath_prepend(str(tmp_path / "src"))
    for name in [m for m in sys.modules if m == "vllm" or m.startswith("vllm.")]:
        monkeypatch.delitem(sys.modules, name)
    mod = importlib.import_module("vllm.v1.attention.backends.triton_attn")
    monkeypatch.setenv(hook.ENABLE_ENV, "1")
    monkeypatch.setenv(hook.FORCE_ENV, "1")
    inp = H.make_synthetic(4, 16, 2, 128, [700, 31, 1500, 64], seed=13, fp8="e5m2")
    kv = torch.stack([inp["key_cache"].view(torch.uint8), inp["value_cache"].view(torch.uint8)])
    impl = mod.TritonAttentionImpl(16, 128, inp["softmax_scale"], 2, kv_cache_dtype="fp8_e5m2")
    layer = types.SimpleNamespace(_k_scale_float=inp["k_scale"], _v_scale_float=inp["v_scale"])
    meta = types.SimpleNamespace(num_actual_tokens=4, query_start_loc=None, seq_lens=inp["seq_lens"],
                                 max_query_len=1, max_seq_len=inp["max_seq_len"], block_table=inp["block_table"])
    out = torch.zeros(4, 16, 128, dtype=torch.bfloat16, device="cuda")
    impl.forward(layer, inp["query"], None, None, kv, meta, output=out)
    torch.cuda.synchronize()
    assert mod.CALLS == []
    exp_out, _ = H.run_oracle(inp)  # e5m2 format (the cache tensors' dtype)
    H.compare(out, None, exp_out, None, check_lse=False)
