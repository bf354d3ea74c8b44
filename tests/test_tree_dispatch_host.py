"""Gates of the tree-attention dispatch helpers (CPU; shapes only, no kernel runs).

The reference's truth table (integrations/vllm/l20_tree_attention_dispatch.py:20-70),
with the device check replaced by gfx950 and head_dim 64 also accepted."""

import pytest
import torch

import l20_tree_attention_dispatch as d


def _t(*shape, dtype=torch.bfloat16):
    return torch.zeros(shape, dtype=dtype)


def _call(draft=4, d_head=128, kv_dtype=torch.bfloat16, page=16, cached=5000, batch=2, suffix_draft=None):
    q = _t(batch, draft, 16, d_head)
    kc = _t(40, page, 4, d_head, dtype=kv_dtype)
    sk = _t(batch, suffix_draft or draft, 4, d_head)
    bt = torch.zeros(batch, 400, dtype=torch.int32)
    return q, kc, sk, bt, cached


@pytest.fixture
def on_mi355x(monkeypatch):
    monkeypatch.setattr(d, "is_mi355x", lambda device=None: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setenv(d.ENABLE_ENV, "1")


def test_off_unless_enabled(monkeypatch):
    monkeypatch.setattr(d, "is_mi355x", lambda device=None: True)
    monkeypatch.delenv(d.ENABLE_ENV, raising=False)
    assert not d.should_dispatch_l20_tree_attention(*_call())
    assert d.maybe_l20_tree_attention(_t(2, 4, 16, 128), None, None, None, None, torch.zeros(2, 4), None, 5000) is None


def test_tree_gate_truth_table(on_mi355x, monkeypatch):
    assert d.should_dispatch_l20_tree_attention(*_call())
    assert d.should_dispatch_l20_tree_attention(*_call(d_head=64))          # MI355X also takes head_dim 64
    assert not d.should_dispatch_l20_tree_attention(*_call(cached=4095))    # the reference's threshold
    assert not d.should_dispatch_l20_tree_attention(*_call(d_head=96))
    assert not d.should_dispatch_l20_tree_attention(*_call(kv_dtype=torch.float16))  # cache dtype != query dtype
    assert not d.should_dispatch_l20_tree_attention(*_call(kv_dtype=torch.float8_e4m3fn))
    assert d.should_dispatch_l20_tree_attention(*_call(page=32))           # pages of any multiple of 16 tokens
    assert d.should_dispatch_l20_tree_attention(*_call(page=64))
    assert not d.should_dispatch_l20_tree_attention(*_call(page=24))
    assert not d.should_dispatch_l20_tree_attention(*_call(page=8))
    assert not d.should_dispatch_l20_tree_attention(*_call(suffix_draft=3))
    q, kc, sk, bt, n = _call()
    assert not d.should_dispatch_l20_tree_attention(q, kc, sk, bt[:1], n)  # batch mismatch
    assert not d.should_dispatch_l20_tree_attention(q.float(), kc, sk, bt, n)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert not d.should_dispatch_l20_tree_attention(*_call())
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(d, "is_mi355x", lambda device=None: False)
    assert not d.should_dispatch_l20_tree_attention(*_call())


def test_causal_verifier_gate(on_mi355x):
    assert d.should_dispatch_l20_causal_verifier_attention(*_call(cached=1024))
    assert not d.should_dispatch_l20_causal_verifier_attention(*_call(cached=1023))
    assert not d.should_dispatch_l20_causal_verifier_attention(*_call(draft=1))
    assert not d.should_dispatch_l20_causal_verifier_attention(*_call(draft=65))
    assert d.should_dispatch_l20_causal_verifier_attention(*_call(draft=64))
