"""Host-side pieces of tree verification: ancestor masks and their 32-bit words."""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "single-gpu-inference-lab_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

import l20_tree_verify as tv  # noqa: E402
from oracle import paged_fp8_decode_ref as ref  # noqa: E402


def test_chain_tree_mask_known_answer():
    """The reference's chain KAT (tests/test_tree_attention.py:14-21)."""
    assert tv.make_chain_tree_mask(4).tolist() == [
        [True, False, False, False],
        [True, True, False, False],
        [True, True, True, False],
        [True, True, True, True],
    ]


@pytest.mark.parametrize("s", [1, 5, 31, 32])
def test_chain_words_closed_form(s):
    """Row i of a chain sees drafts 0..i: word 2^(i+1) - 1 (as int32)."""
    w = tv.tree_mask_bits(tv.make_chain_tree_mask(s)).to(torch.int64) & 0xFFFFFFFF
    assert w.tolist() == [(1 << (i + 1)) - 1 for i in range(s)]


def test_words_match_oracle_and_bit31():
    rng = np.random.default_rng(0)
    m = rng.random((3, 32, 32)) < 0.4
    m[0, 5, 31] = True
    got = tv.tree_mask_bits(torch.from_numpy(m))
    assert got.dtype == torch.int32 and got.shape == (3, 32)
    exp = ref.tree_bits_from_mask(m)
    assert np.array_equal(got.numpy().astype(np.int64) & 0xFFFFFFFF, exp)
    assert got[0, 5].item() < 0  # bit 31 shows as the int32 sign


def test_words_visibility_round_trip():
    """Words decoded by the oracle's visibility rule give back the mask's draft columns."""
    rng = np.random.default_rng(1)
    s, length = 7, 20
    m = rng.random((s, s)) < 0.5
    vis = ref.tree_visibility(length, s, tv.tree_mask_bits(torch.from_numpy(m)).numpy())
    assert vis[:, : length - s].all()
    assert np.array_equal(vis[:, length - s:], m)


def test_words_reject_bad_shapes():
    with pytest.raises(ValueError):
        tv.tree_mask_bits(torch.ones(3, 4, dtype=torch.bool))
    with pytest.raises(ValueError):
        tv.tree_mask_bits(torch.ones(33, 33, dtype=torch.bool))


def test_workspace_layout():
    q = torch.zeros(2, 5, 8, 64)
    ws = tv.allocate_tree_attention_workspace(q)
    assert [tuple(t.shape) for t in ws] == [(2, 5, 8, 64), (2, 5, 8), (2, 5, 8)] * 2
    assert all(t.dtype == torch.float32 for t in ws)


def test_reference_policy_helpers():
    import l20_tree_verify as tv

    # the split form is the only MI355X tree path; the tile policy keeps the reference's values
    assert all(tv.should_use_l20_split_tree_attention(n) for n in (0, 1, 4095, 4096, 131072))
    assert [tv.l20_tree_attention_block_t(n) for n in (0, 4095, 4096, 100000)] == [64, 64, 128, 128]
    for n in (0, 4095, 4096):
        tv._check_block_t(tv.l20_tree_attention_block_t(n))  # accepted by the entry points
