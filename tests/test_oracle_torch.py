"""Pins for the torch CPU restatement (oracle/paged_fp8_decode_torch.py), the
CPU baseline bench.py times: it must agree with the pinned numpy oracle on
every feature it handles (CPU only)."""

import numpy as np
import pytest
import torch

from oracle import paged_fp8_decode_ref as ref
from oracle import paged_fp8_decode_torch as tref


def _case(seed, batch, hq, hkv, d, lens, q_len=1, per_head=False, kv16=None, tree=False):
    g = torch.Generator().manual_seed(seed)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    pages_per = (lens_t.long() + 15) // 16
    pool = int(pages_per.sum()) + 5
    perm = torch.randperm(pool, generator=g)
    table = torch.full((batch, max(1, int(pages_per.max()))), -1, dtype=torch.int32)
    off = 0
    for b in range(batch):
        n = int(pages_per[b])
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    query = torch.randn(batch * q_len, hq, d, generator=g).to(torch.bfloat16)
    caches, scales = [], []
    for _ in range(2):
        raw = torch.randn(pool, 16, hkv, d, generator=g)
        if kv16 is not None:
            caches.append(raw.to(kv16))
            scales.append(1.0)
        elif per_head:
            c, s = ref.quantize_fp8_e4m3_per_head(raw.numpy())
            caches.append(torch.from_numpy(c).view(torch.float8_e4m3fn))
            scales.append(torch.from_numpy(s))
        else:
            c, s = ref.quantize_fp8_e4m3(raw.numpy())
            caches.append(torch.from_numpy(c).view(torch.float8_e4m3fn))
            scales.append(s)
    words = None
    if tree:
        words = torch.randint(0, 2 ** q_len, (batch, q_len), generator=g, dtype=torch.int64)
        words |= 1 << torch.arange(q_len)  # a row sees its own draft
        words = words.to(torch.int32)
    return dict(query=query, key_cache=caches[0], value_cache=caches[1], block_table=table, seq_lens=lens_t,
                k_scale=scales[0], v_scale=scales[1], q_len=q_len, tree_mask=words)


def _numpy_oracle(c):
    def sc(x):
        return x.numpy() if isinstance(x, torch.Tensor) else x

    q = c["query"].float().numpy()
    tree = None if c["tree_mask"] is None else c["tree_mask"].numpy().astype(np.int64)
    if c["key_cache"].dtype == torch.float8_e4m3fn:
        return ref.reference(q, c["key_cache"].view(torch.uint8).numpy(), c["value_cache"].view(torch.uint8).numpy(),
                             c["block_table"].numpy(), c["seq_lens"].numpy(), sc(c["k_scale"]), sc(c["v_scale"]),
                             q_len=c["q_len"], tree_mask=tree)
    return ref.reference_dense_kv(q, c["key_cache"].float().numpy(), c["value_cache"].float().numpy(),
                                  c["block_table"].numpy(), c["seq_lens"].numpy(), q_len=c["q_len"], tree_mask=tree)


CASES = [
    dict(seed=1, batch=3, hq=14, hkv=2, d=64, lens=[17, 300, 64]),
    dict(seed=2, batch=2, hq=28, hkv=4, d=128, lens=[1, 513], per_head=True),
    dict(seed=3, batch=2, hq=16, hkv=2, d=128, lens=[70, 4], q_len=4),
    dict(seed=4, batch=2, hq=8, hkv=2, d=64, lens=[2, 40], q_len=4, per_head=True),   # rows without keys
    dict(seed=5, batch=3, hq=16, hkv=2, d=128, lens=[0, 33, 100]),                   # empty sequence
    dict(seed=6, batch=2, hq=16, hkv=8, d=128, lens=[90, 37], q_len=4, tree=True),
    dict(seed=7, batch=2, hq=16, hkv=2, d=128, lens=[90, 300], kv16=torch.bfloat16),
    dict(seed=8, batch=2, hq=8, hkv=2, d=64, lens=[45, 3], q_len=2, kv16=torch.float16),
]


@pytest.mark.parametrize("spec", CASES)
def test_torch_restatement_matches_numpy_oracle(spec):
    c = _case(**spec)
    want_out, want_lse = _numpy_oracle(c)
    out, lse = tref.reference_torch(c["query"], c["key_cache"], c["value_cache"], c["block_table"], c["seq_lens"],
                                    c["k_scale"], c["v_scale"], q_len=c["q_len"], tree_mask=c["tree_mask"])
    np.testing.assert_allclose(out.numpy(), want_out, atol=2e-6, rtol=0)
    finite = np.isfinite(want_lse)
    assert np.array_equal(np.isfinite(lse.numpy()), finite)
    np.testing.assert_allclose(lse.numpy()[finite], want_lse[finite], atol=2e-6, rtol=0)
