"""Rounding of the softmax probabilities on the MFMA path (GPU).

The P.V product takes P in the MFMA operand type (f16 for fp8 caches, the
cache type for 16-bit ones) while the softmax denominator sums P unrounded.
When many keys share one probability that the operand type cannot hold, the
rounding of P is the same for all of them and does not average out over a
long context.  These cases make that bias large: every other key scores
Delta = 0.0996 (log2 units) below its neighbours, so its probability
2^-Delta = 0.93329 is not an f16 (or bf16) value, and V is +-448 (the largest
e4m3fn value) on alternating keys, so the output (~15.5) is the small
difference of two large sums.  A P rounded once to 11 bits missed the oracle
by 0.033 here on MI355X (more than the 1e-2 tolerance); split into hi + lo it
meets the closed form below to the output's own rounding.  Queries and
outputs are fp16, whose rounding of ~15.5 is below 3.9e-3.

The output has a closed form: with n equal even and odd keys, probability
p = 2^-Delta for the odd ones, out = 448 (1 - p) / (1 + p) in every dimension
and lse = s_even + ln(n (1 + p)).  The test pins the op to that float64 value
within the fp16 half-ulp at 15.5 (3.9e-3), which a P rounded once misses
(0.03), and to the fp32 oracle (oracle/paged_fp8_decode_ref.py) at the usual
tolerances (max-abs 1e-2, cosine 0.9999, LSE 1e-4 relative); the oracle's own
fp32 sum of 32768 terms of +-448 is 5e-3 off the closed form here, which is
why the tight bound uses the closed form.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu

L = 32768          # one long sequence: 2048 pages, 32 to 64 splits
HQ, HKV, D = 8, 1, 128
Q0 = 6.25          # query = Q0 * e_0; score gap Q0 * 0.125 * D^-0.5 * log2(e) = 0.0996


def adversarial(kv: str):
    """One sequence of L tokens: keys 1.0 / 0.875 along dim 0, values +448 / -448."""
    g = torch.Generator().manual_seed(5)
    pages = L // 16
    perm = torch.randperm(pages + 3, generator=g)[:pages].to(torch.int32)
    table = perm.view(1, pages)
    tok = torch.arange(L)
    key = torch.zeros(pages + 3, 16, HKV, D)
    val = torch.zeros(pages + 3, 16, HKV, D)
    kvals = torch.where(tok % 2 == 0, 1.0, 0.875)
    vvals = torch.where(tok % 2 == 0, 448.0, -448.0)
    key.view(-1, HKV, D)[perm.long().repeat_interleave(16) * 16 + tok % 16, 0, 0] = kvals
    val.view(-1, HKV, D)[perm.long().repeat_interleave(16) * 16 + tok % 16, 0, :] = vvals[:, None]
    query = torch.zeros(1, HQ, D)
    query[0, :, 0] = Q0
    inp = {
        "query": query.to(torch.float16).cuda(), "block_table": table.cuda(),
        "seq_lens": torch.tensor([L], dtype=torch.int32).cuda(), "softmax_scale": D ** -0.5,
        "q_len": 1, "max_seq_len": L,
    }
    if kv == "fp8":
        inp.update(key_cache=key.to(torch.float8_e4m3fn).cuda(), value_cache=val.to(torch.float8_e4m3fn).cuda(),
                   k_scale=1.0, v_scale=1.0)
    else:
        inp.update(key_cache=key.to(torch.float16).cuda(), value_cache=val.to(torch.float16).cuda())
    return inp


@pytest.mark.parametrize("kv", ["fp8", "fp16"])
@pytest.mark.parametrize("split", [512, 1024])
def test_probability_rounding_does_not_bias_long_contexts(kv, split):
    inp = adversarial(kv)
    if kv == "fp8":
        out, lse = H.run_op(inp, split)
        exp_out, exp_lse = H.run_oracle(inp)
    else:
        out, lse = H.run_op16(inp, split)
        exp_out, exp_lse = H.run_oracle16(inp)
    H.compare(out, lse, exp_out, exp_lse)
    s_even = Q0 * D ** -0.5                       # natural-log score of the even keys
    p = np.exp(Q0 * (0.875 - 1.0) * D ** -0.5)    # odd keys' probability relative to even ones
    exact = 448.0 * (1.0 - p) / (1.0 + p)
    exact_lse = s_even + np.log((L // 2) * (1.0 + p))
    assert 15.0 < exact < 16.0                    # the case is what it claims: a small difference of large sums
    err = float(np.abs(out.float().cpu().numpy() - exact).max())
    assert err < 3.9e-3, err
    assert float(np.abs(lse.cpu().numpy() - exact_lse).max()) < 1e-5 * exact_lse
