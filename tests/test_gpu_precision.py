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


SPIKE_L = 600      # 19 blocks of 32 tokens, two 512-token splits
SPIKE_B = 32       # one sequence per token position inside a 32-token block


def spiky(kv: str, q_len: int):
    """Sequence b holds one spike key at position b of every 32-token block.

    The spike keys score ~30 log2 units above the rest (key 16.0 against keys
    in [-1, 1] along the query's one non-zero dimension), so a block's maximum
    sits in whichever lane row holds position b.  A maximum reduced over only
    some lane rows leaves the spikes' probabilities at ~2^30, far past f16's
    range, and the output turns inf/NaN; the exact maximum gives the mean of
    the spikes' values.
    """
    g = torch.Generator().manual_seed(11)
    per = (SPIKE_L + 15) // 16
    pages = SPIKE_B * per
    perm = torch.randperm(pages + 5, generator=g)[:pages].to(torch.int32)
    table = perm.view(SPIKE_B, per)
    key = torch.zeros(pages + 5, 16, HKV, D)
    val = torch.zeros(pages + 5, 16, HKV, D)
    tok = torch.arange(SPIKE_L)
    for b in range(SPIKE_B):
        slots = table[b].long().repeat_interleave(16)[:SPIKE_L] * 16 + tok % 16
        k0 = torch.rand(SPIKE_L, generator=g) * 2.0 - 1.0
        k0[tok % 32 == b] = 16.0
        key.view(-1, HKV, D)[slots, 0, 0] = k0
        val.view(-1, HKV, D)[slots, 0, :] = torch.rand(SPIKE_L, D, generator=g) * 8.0 - 4.0
    query = torch.zeros(SPIKE_B * q_len, HQ, D)
    query[:, :, 0] = 16.0
    inp = {
        "query": query.to(torch.float16).cuda(), "block_table": table.cuda(),
        "seq_lens": torch.full((SPIKE_B,), SPIKE_L, dtype=torch.int32).cuda(), "softmax_scale": D ** -0.5,
        "q_len": q_len, "max_seq_len": SPIKE_L,
    }
    if kv == "fp8":
        inp.update(key_cache=key.to(torch.float8_e4m3fn).cuda(), value_cache=val.to(torch.float8_e4m3fn).cuda(),
                   k_scale=1.0, v_scale=1.0)
    else:
        inp.update(key_cache=key.to(torch.float16).cuda(), value_cache=val.to(torch.float16).cuda())
    return inp


@pytest.mark.parametrize("kv", ["fp8", "fp16"])
@pytest.mark.parametrize("q_len", [1, 4])
@pytest.mark.parametrize("split", [256, 512])
def test_block_maximum_covers_every_lane_row(kv, q_len, split):
    inp = spiky(kv, q_len)
    if kv == "fp8":
        out, lse = H.run_op(inp, split)
        exp_out, exp_lse = H.run_oracle(inp)
    else:
        out, lse = H.run_op16(inp, split)
        exp_out, exp_lse = H.run_oracle16(inp)
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
    H.compare(out, lse, exp_out, exp_lse)
    # Closed form: the other keys weigh < 600 * 2^-28 against a spike, so each
    # query row's output is the mean of the values of the spikes it can see.
    vc = inp["value_cache"].float().cpu().view(-1, HKV, D)
    table = inp["block_table"].cpu().long()
    got = out.float().cpu().view(SPIKE_B, q_len, HQ, D)
    for b in range(SPIKE_B):
        for i in range(q_len):
            seen = torch.arange(b, SPIKE_L - q_len + i + 1, 32)
            spikes = vc[table[b, seen // 16] * 16 + seen % 16, 0]
            err = float((got[b, i] - spikes.mean(0)).abs().max())
            assert err < 2e-2, (b, i, err)
