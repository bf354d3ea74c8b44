"""The vLLM ROCm install hook: installer on a stand-in vLLM tree (text fixture)
and the dispatch gates (CPU); the GPU run of the patched forward is in
test_gpu_vllm_rocm_hook.py."""

import importlib
import py_compile
import shutil
import sys
import types
from pathlib import Path

import pytest
import torch

import install_l20_fp8_paged_decode_rocm as inst
import l20_vllm_rocm_hook as hook

FIXTURE = Path(__file__).parent / "fixtures" / "vllm_rocm"


@pytest.fixture
def vllm_tree(tmp_path):
    shutil.copytree(FIXTURE, tmp_path / "src")
    return tmp_path / "src"


def test_install_patches_once_and_uninstall_restores(vllm_tree):
    package = inst.find_vllm_package(str(vllm_tree))
    backend = package / inst.BACKEND
    original = backend.read_text()
    assert inst.main(["--vllm-source-dir", str(vllm_tree)]) == 0
    patched = backend.read_text()
    assert patched.count("l20_fp8_paged_decode_or_none(self, layer") == 1
    assert patched.index("l20_fp8_paged_decode_or_none(self") < patched.index("        unified_attention(")
    py_compile.compile(str(backend), doraise=True)
    shim = (package / inst.SHIM).read_text()
    assert str(inst.HERE) in shim and "l20_fp8_paged_decode_or_none" in shim
    # idempotent
    inst.main(["--vllm-source-dir", str(vllm_tree)])
    assert backend.read_text() == patched
    inst.main(["--vllm-source-dir", str(vllm_tree), "--uninstall"])
    assert backend.read_text() == original
    assert not (package / inst.SHIM).exists()
    assert not backend.with_suffix(inst.BACKUP_SUFFIX).exists()


def test_missing_patch_point_is_an_error(vllm_tree):
    backend = vllm_tree / "vllm" / inst.BACKEND
    backend.write_text(backend.read_text().replace("unified_attention(\n            q=", "other_attention(\n            q="))
    with pytest.raises(RuntimeError, match="cannot find patch point"):
        inst.main(["--vllm-source-dir", str(vllm_tree)])


def test_cannot_find_package(tmp_path):
    with pytest.raises(RuntimeError, match="cannot find vLLM source package"):
        inst.find_vllm_package(str(tmp_path))


def test_gates_use_the_reference_environment_names():
    source = Path(hook.__file__).read_text()
    for name in ("VLLM_ENABLE_L20_FP8_PAGED_DECODE", "VLLM_L20_FP8_PAGED_FORCE", "VLLM_L20_FP8_PAGED_TRACE",
                 "should_use_l20_paged_fp8_split_kv", "l20_paged_split_kv_attention_fp8",
                 "allocate_l20_paged_split_kv_workspace"):
        assert name in source


def _fake_call(batch=4, hq=16, hkv=2, d=128, max_query_len=1, kv_dtype="fp8"):
    impl = types.SimpleNamespace(kv_cache_dtype=kv_dtype, alibi_slopes=None, sliding_window=(-1, -1),
                                 logits_soft_cap=0, sinks=None, scale=d ** -0.5)
    layer = types.SimpleNamespace(_k_scale_float=0.1, _v_scale_float=0.1)
    query = torch.zeros(batch, hq, d, dtype=torch.bfloat16)
    kc = torch.zeros(10, 16, hkv, d, dtype=torch.float8_e4m3fn)
    meta = types.SimpleNamespace(max_query_len=max_query_len, max_seq_len=100,
                                 block_table=torch.zeros(batch, 7, dtype=torch.int32),
                                 seq_lens=torch.full((batch,), 100, dtype=torch.int32))
    return impl, layer, query, kc, kc.clone(), meta, batch


def test_gate_rejects_each_unsupported_case(monkeypatch):
    import l20_paged_split_kv

    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    impl, layer, q, kc, vc, meta, n = _fake_call()
    monkeypatch.delenv(hook.ENABLE_ENV, raising=False)
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n)  # off by default
    monkeypatch.setenv(hook.ENABLE_ENV, "1")
    assert hook.decode_gate(impl, layer, q, kc, vc, meta, n)
    cases = [
        dict(kv_dtype="auto"),              # not an fp8 cache
        dict(max_query_len=2),              # prefill / mixed batch
        dict(d=96),                         # head size
    ]
    for kw in cases:
        args = _fake_call(**kw)
        assert not hook.decode_gate(*args), kw
    for attr, value in (("alibi_slopes", torch.ones(16)), ("sliding_window", (128, 0)), ("logits_soft_cap", 30.0),
                        ("sinks", torch.zeros(16))):
        impl2 = types.SimpleNamespace(**vars(impl))
        setattr(impl2, attr, value)
        assert not hook.decode_gate(impl2, layer, q, kc, vc, meta, n), attr
    assert not hook.decode_gate(impl, layer, q, kc.view(torch.int8), vc, meta, n)  # not a byte view of fp8 codes
    assert not hook.decode_gate(*_fake_call(kv_dtype="fp8_e4m3fnuz"))  # a format the op does not read
    # e5m2 caches take the path; vLLM's backend hands them over viewed as its platform type
    assert hook.decode_gate(*_fake_call(kv_dtype="fp8_e5m2"))
    assert hook.cache_format(types.SimpleNamespace(kv_cache_dtype="fp8_e5m2")) == torch.float8_e5m2
    for kind in ("fp8", "fp8_e4m3"):
        assert hook.cache_format(types.SimpleNamespace(kv_cache_dtype=kind)) == torch.float8_e4m3fn
    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: False)
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n)  # not gfx950
    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n)  # graph capture


def test_patched_forward_falls_back_when_disabled(vllm_tree, monkeypatch):
    """The patched stand-in forward runs vLLM's kernel when the gate is closed."""
    inst.main(["--vllm-source-dir", str(vllm_tree)])
    monkeypatch.syspath_prepend(str(vllm_tree))
    monkeypatch.delenv(hook.ENABLE_ENV, raising=False)
    for name in [m for m in sys.modules if m == "vllm" or m.startswith("vllm.")]:
        monkeypatch.delitem(sys.modules, name)
    mod = importlib.import_module("vllm.v1.attention.backends.triton_attn")
    impl = mod.TritonAttentionImpl(16, 128, 128 ** -0.5, 2)
    layer = types.SimpleNamespace(_k_scale_float=1.0, _v_scale_float=1.0)
    kv = torch.zeros(2, 10, 16, 2, 128, dtype=torch.uint8)
    meta = types.SimpleNamespace(num_actual_tokens=3, query_start_loc=None, seq_lens=torch.ones(3, dtype=torch.int32),
                                 max_query_len=1, max_seq_len=1, block_table=torch.zeros(3, 1, dtype=torch.int32))
    q = torch.zeros(3, 16, 128, dtype=torch.bfloat16)
    out = torch.zeros_like(q)
    impl.forward(layer, q, None, None, kv, meta, output=out)
    assert len(mod.CALLS) == 1 and bool((out == -1).all())


def test_heuristic_gates_stay_closed_for_every_shape(monkeypatch):
    """The reference's policy test (tests/test_l20_paged_split_kv_policy.py:20-43):
    both heuristic gates are False for every shape, also on an MI355X."""
    import l20_paged_split_kv

    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: True)
    for batch, max_seq in ((1, 2048), (1, 4096), (4, 4096), (8, 2048), (8, 4096), (128, 8192), (0, 0)):
        assert l20_paged_split_kv.should_use_l20_paged_fp8_split_kv(batch, max_seq) is False
        assert l20_paged_split_kv.should_use_l20_paged_split_kv(batch, max_seq) is False


def test_dispatch_truth_table(monkeypatch):
    """ENABLE x FORCE: only ENABLE=1 with FORCE=1 reaches the op (the heuristic gate is closed)."""
    import l20_paged_split_kv

    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    ran = []
    monkeypatch.setattr(l20_paged_split_kv, "l20_paged_split_kv_attention_fp8", lambda *a, **k: ran.append(k))
    monkeypatch.setattr(l20_paged_split_kv, "allocate_l20_paged_split_kv_workspace", lambda *a, **k: None)
    impl, layer, q, kc, vc, meta, n = _fake_call()
    out = torch.zeros_like(q)
    for enable in ("0", "1"):
        for force in ("0", "1"):
            monkeypatch.setenv(hook.ENABLE_ENV, enable)
            monkeypatch.setenv(hook.FORCE_ENV, force)
            ran.clear()
            took = hook.l20_fp8_paged_decode_or_none(impl, layer, q, kc, vc, out, meta, n)
            assert took == (enable == "1" and force == "1"), (enable, force)
            assert len(ran) == int(took)


def test_gate_rejects_quantised_or_mismatched_output(monkeypatch):
    import l20_paged_split_kv

    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setenv(hook.ENABLE_ENV, "1")
    impl, layer, q, kc, vc, meta, n = _fake_call()
    assert hook.decode_gate(impl, layer, q, kc, vc, meta, n, output=torch.zeros_like(q))
    assert hook.decode_gate(impl, layer, q, kc, vc, meta, n, output=torch.zeros(n, 16 * 128, dtype=q.dtype))
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n, output=torch.zeros_like(q),
                                output_scale=torch.ones(()))
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n,
                                output=torch.zeros(q.shape, dtype=torch.float8_e4m3fn))
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n, output=torch.zeros(q.shape, dtype=torch.float16))
    assert not hook.decode_gate(impl, layer, q, kc, vc, meta, n, output=torch.zeros(n - 1, 16, 128, dtype=q.dtype))


@pytest.mark.parametrize("case", ["output_scale", "fp8_output"])
def test_patched_forward_falls_back_on_quantised_output(vllm_tree, monkeypatch, case):
    """With every env gate open (ENABLE and FORCE) and a GPU stand-in, a fused
    output quantisation still reaches vLLM's own kernel (the stub)."""
    import l20_paged_split_kv

    inst.main(["--vllm-source-dir", str(vllm_tree)])
    monkeypatch.syspath_prepend(str(vllm_tree))
    monkeypatch.setenv(hook.ENABLE_ENV, "1")
    monkeypatch.setenv(hook.FORCE_ENV, "1")
    monkeypatch.setattr(l20_paged_split_kv, "is_mi355x", lambda device=None: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)

    def must_not_run(*a, **k):
        raise AssertionError("the MI355X op must not run for a quantised output")

    monkeypatch.setattr(l20_paged_split_kv, "l20_paged_split_kv_attention_fp8", must_not_run)
    for name in [m for m in sys.modules if m == "vllm" or m.startswith("vllm.")]:
        monkeypatch.delitem(sys.modules, name)
    mod = importlib.import_module("vllm.v1.attention.backends.triton_attn")
    impl = mod.TritonAttentionImpl(16, 128, 128 ** -0.5, 2, kv_cache_dtype="fp8_e4m3")
    layer = types.SimpleNamespace(_k_scale_float=1.0, _v_scale_float=1.0)
    kv = torch.zeros(2, 10, 16, 2, 128, dtype=torch.uint8)
    meta = types.SimpleNamespace(num_actual_tokens=3, query_start_loc=None, seq_lens=torch.ones(3, dtype=torch.int32),
                                 max_query_len=1, max_seq_len=1, block_table=torch.zeros(3, 1, dtype=torch.int32))
    q = torch.zeros(3, 16, 128, dtype=torch.bfloat16)
    if case == "output_scale":
        out = torch.zeros_like(q)
        impl.forward(layer, q, None, None, kv, meta, output=out, output_scale=torch.ones(()))
    else:
        out = torch.zeros(3, 16, 128, dtype=torch.float8_e4m3fn)
        impl.forward(layer, q, None, None, kv, meta, output=out)
    assert len(mod.CALLS) == 1
