"""CPU pin of the tree-attention checkers used by the GPU tree tests.

``pd_helpers.dense_tree_oracle`` (an fp64 restatement over concatenated prefix and
draft keys) against ``pd_helpers.paged_tree_oracle`` (the oracle's
``reference_dense_kv`` with tree words, keys laid out as pages; itself pinned in
test_oracle.py), on tree masks of 5-32 drafts (the oracle's tree words are 32
bits, like the kernels'; the dense restatement's formula does not depend on the
draft count) and 16/32-token pages; planted mistakes (a transposed mask, a
dropped prefix) must be caught.
"""

from __future__ import annotations

import numpy as np
import pytest

import pd_helpers as H


def _tree(s, rng):
    """Random ancestor mask: each draft's parent is an earlier draft (or the root)."""
    parent = [-1] + [int(rng.integers(-1, i)) for i in range(1, s)]
    m = np.zeros((s, s), dtype=bool)
    for i in range(s):
        j = i
        while j >= 0:
            m[i, j] = True
            j = parent[j]
    return m


def _case(b, s, hq, hkv, d, cached, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, s, hq, d)).astype(np.float32)
    pk = rng.standard_normal((b, cached, hkv, d)).astype(np.float32)
    pv = rng.standard_normal((b, cached, hkv, d)).astype(np.float32)
    sk = rng.standard_normal((b, s, hkv, d)).astype(np.float32)
    sv = rng.standard_normal((b, s, hkv, d)).astype(np.float32)
    return q, pk, pv, sk, sv, _tree(s, rng)


@pytest.mark.parametrize("b,s,hq,hkv,d,cached,page", [
    (2, 5, 4, 2, 64, 37, 16),
    (1, 32, 4, 4, 64, 20, 16),     # a full 32-bit word of drafts
    (2, 8, 8, 2, 128, 0, 16),      # no cached prefix
    (2, 6, 4, 1, 64, 70, 32),
])
def test_dense_tree_oracle_equals_paged_reference(b, s, hq, hkv, d, cached, page):
    q, pk, pv, sk, sv, mask = _case(b, s, hq, hkv, d, cached, seed=s * 7 + cached)
    scale = d ** -0.5
    dense = H.dense_tree_oracle(q, pk, pv, sk, sv, mask, scale)
    out, lse = H.paged_tree_oracle(q, pk, pv, sk, sv, mask, scale, page=page)
    np.testing.assert_allclose(out, dense, atol=2e-6, rtol=1e-5)
    assert np.isfinite(lse).all()
    # planted mistakes: the mask transposed, the prefix dropped
    wrong_t = H.dense_tree_oracle(q, pk, pv, sk, sv, mask.T, scale)
    assert not np.allclose(wrong_t, out, atol=1e-3)
    if cached:
        wrong_p = H.dense_tree_oracle(q, pk[:, :0], pv[:, :0], sk, sv, mask, scale)
        assert not np.allclose(wrong_p, out, atol=1e-3)


def test_prefix_only_lse_is_the_logsumexp_of_the_prefix_scores():
    """With an all-False mask every row sees the prefix alone: the LSE is the
    closed-form logsumexp of its prefix scores (what the hybrid path's prefix pass
    returns)."""
    b, s, hq, hkv, d, cached = 2, 4, 4, 2, 64, 29
    q, pk, pv, sk, sv, _ = _case(b, s, hq, hkv, d, cached, seed=3)
    none = np.zeros((s, s), dtype=bool)
    scale = d ** -0.5
    _, lse = H.paged_tree_oracle(q, pk, pv, sk, sv, none, scale)
    g = hq // hkv
    for i in range(b):
        for r in range(s):
            for h in range(hq):
                sc = pk[i, :, h // g].astype(np.float64) @ q[i, r, h].astype(np.float64) * scale
                want = sc.max() + np.log(np.exp(sc - sc.max()).sum())
                assert abs(lse[i, r, h] - want) <= 1e-5 * max(1.0, abs(want))
