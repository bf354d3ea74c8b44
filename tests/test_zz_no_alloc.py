"""GPU: the allocation-free entry point ``l20_pd_fp8_e4m3_split_out_noalloc``
(split partials in the library's per-device scratch) against
``l20_pd_fp8_e4m3_split_out`` with a caller workspace, through the C ABI."""

import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    import l20_paged_decode  # noqa: F401  (fails loudly if the extension is missing)


def run_noalloc(inp, split):
    import l20_pd_cabi as cabi

    q = inp["query"]
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[0], q.shape[1], dtype=torch.float32, device=q.device)
    ks, ksph = H._scales(inp["k_scale"])
    vs, vsph = H._scales(inp["v_scale"])
    args = cabi.args_from_tensors(q, inp["key_cache"], inp["value_cache"], inp["block_table"], inp["seq_lens"],
                                  None, None, None, out, ks, vs, inp["max_seq_len"], split,
                                  softmax_scale=inp["softmax_scale"], k_scale_per_head=ksph,
                                  v_scale_per_head=vsph, q_len=inp["q_len"], lse=lse)
    cabi.split_out_noalloc(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, lse


def test_noalloc_matches_the_workspace_entry_point_on_two_calls():
    """A large call, then a smaller one whose partial layout differs (the
    scratch still holds the first call's partials): both bitwise equal to the
    caller-workspace entry point and within tolerance of the oracle."""
    big = H.make_synthetic(8, 28, 4, 128, [5000, 17, 1025, 3000, 512, 4097, 64, 2048], seed=71)
    small = H.make_synthetic(3, 16, 2, 64, [700, 100, 33], q_len=2, per_head=True, dtype=torch.float16, seed=72)
    for inp, split in ((big, 512), (small, 128)):
        print("noalloc case", inp["query"].shape, split, flush=True)
        want = H.run_op(inp, split, via="cabi")
        got = run_noalloc(inp, split)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        H.compare(*got, *H.run_oracle(inp))


def test_noalloc_single_split_needs_no_scratch():
    inp = H.make_synthetic(4, 14, 2, 64, [64, 200, 511, 17], seed=73)
    want = H.run_op(inp, 1024, via="cabi")
    got = run_noalloc(inp, 1024)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_noalloc_rejects_partials_beyond_the_scratch():
    """128 sequences x 28 heads x 128 splits of 130 fp32 words = 238 MB > 64 MiB."""
    import l20_pd_cabi as cabi

    inp = H.make_synthetic(128, 28, 4, 128, [16] * 127 + [8192], seed=74)
    with pytest.raises(RuntimeError, match="noalloc: the split partials need .* more than the 67108864-byte"):
        run_noalloc(inp, 64)
    # nothing was enqueued: the device is still usable and the next call works
    got = run_noalloc(inp, 1024)
    want = H.run_op(inp, 1024, via="cabi")
    assert torch.equal(got[0], want[0])
    assert cabi.last_error() == ""
