"""GPU parity of speculative tree verification (ancestor bitmasks over the newest
q_len keys) on the streaming split-KV kernel, against the CPU oracle.

Visibility (``triton_tree_attention.py:1218-1240`` of the reference): draft row
i sees the cached prefix and draft j iff ``ancestor_mask[i, j]``.  Tolerances
are the decode parity tolerances of ``pd_helpers``.
"""

import numpy as np
import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu


def random_tree(s, rng):
    """Ancestor mask of a random tree over s drafts (parent index < child index)."""
    parent = [-1] + [int(rng.integers(-1, i)) for i in range(1, s)]
    m = np.zeros((s, s), dtype=bool)
    for i in range(s):
        j = i
        while j >= 0:
            m[i, j] = True
            j = parent[j]
    return m


def words(mask):
    from oracle import paged_fp8_decode_ref as ref

    w = ref.tree_bits_from_mask(mask)
    return torch.from_numpy(np.where(w >= 2**31, w - 2**32, w).astype(np.int32))


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


TREE_SHAPES = [
    # batch, hq, hkv, d, lens, q_len, split
    (3, 8, 2, 128, [700, 37, 1500], 4, 256),     # 16 columns
    (2, 16, 2, 128, [1000, 333], 4, 512),        # 32 columns (two 16-column tiles)
    (2, 32, 32, 64, [530, 64], 8, 128),          # MHA, d=64
    (2, 4, 4, 128, [900, 32], 32, 256),          # 32 drafts, group 1, one sequence all drafts
    (4, 28, 4, 128, [2048, 17, 300, 4], 4, 512),  # Qwen-7B heads; one sequence holds only its drafts
    (3, 64, 8, 128, [4096, 1500, 9], 4, 1024),   # verify heads, 1024-token splits (one block in flight)
]


@pytest.mark.parametrize("shape", TREE_SHAPES, ids=[f"t{i}" for i in range(len(TREE_SHAPES))])
@pytest.mark.parametrize("via", ["torch", "cabi"])
def test_fp8_tree_mask_matches_oracle(shape, via):
    batch, hq, hkv, d, lens, q_len, split = shape
    print(f"fp8 tree {shape} via={via}", flush=True)
    rng = np.random.default_rng(len(lens) * 31 + q_len)
    inp = H.make_synthetic(batch, hq, hkv, d, lens, q_len=q_len, seed=7 + q_len, garbage_tail=True)
    masks = np.stack([random_tree(q_len, rng) for _ in range(batch)])
    inp["tree_mask"] = words(masks).cuda()
    out, lse = H.run_op(inp, split, via=via)
    exp_out, exp_lse = H.run_oracle(inp)
    H.compare(out, lse, exp_out, exp_lse)


def test_fp8_tree_shared_mask_and_arbitrary_bits():
    """A [q_len] mask shared by the batch, with words that are not tree-shaped
    (bit 31 set, rows seeing no draft at all)."""
    q_len = 32
    inp = H.make_synthetic(2, 4, 4, 128, [1200, 40], q_len=q_len, seed=3)
    rng = np.random.default_rng(5)
    w = rng.integers(0, 2**32, size=q_len, dtype=np.int64)
    w[0] = 0
    w[1] = 2**31
    w[2] = 2**32 - 1
    inp["tree_mask"] = torch.from_numpy(np.where(w >= 2**31, w - 2**32, w).astype(np.int32)).cuda()
    out, lse = H.run_op(inp, 256)
    exp_out, exp_lse = H.run_oracle(inp)
    H.compare(out, lse, exp_out, exp_lse)


def test_fp8_chain_tree_equals_causal():
    """The chain mask reproduces the causal verifier bit for bit."""
    q_len = 8
    inp = H.make_synthetic(3, 32, 8, 128, [3000, 600, 8], q_len=q_len, seed=11)
    base_out, base_lse = H.run_op(inp, 512)
    chain = np.tril(np.ones((q_len, q_len), dtype=bool))
    inp["tree_mask"] = words(chain).cuda()
    out, lse = H.run_op(inp, 512)
    assert torch.equal(out, base_out)
    assert torch.equal(lse, base_lse)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("csr", [False, True])
def test_16bit_tree_mask_matches_oracle(dtype, csr):
    print(f"16-bit tree dtype={dtype} csr={csr}", flush=True)
    q_len = 6
    rng = np.random.default_rng(17)
    inp = H.make_synthetic16(3, 20, 4, 128, [800, 6, 2100], dtype=dtype, q_len=q_len, seed=23,
                             garbage_tail=True, csr_pad=2 if csr else 0)
    masks = np.stack([random_tree(q_len, rng) for _ in range(3)])
    inp["tree_mask"] = words(masks).cuda()
    out, lse = H.run_op16(inp, 512, csr=csr, via="cabi" if csr else "torch")
    exp_out, exp_lse = H.run_oracle16(inp, csr=csr)
    H.compare(out, lse, exp_out, exp_lse)


def test_tree_mask_rejects_bad_shapes():
    inp = H.make_synthetic(2, 8, 2, 128, [100, 50], q_len=4, seed=1)
    inp["tree_mask"] = torch.zeros(3, 4, dtype=torch.int32, device="cuda")  # wrong batch
    with pytest.raises(RuntimeError, match="tree_mask"):
        H.run_op(inp, 256)
    inp["tree_mask"] = torch.zeros(2, 4, dtype=torch.int64, device="cuda")  # wrong dtype
    with pytest.raises(RuntimeError, match="tree_mask"):
        H.run_op(inp, 256)


# ------------------------------------------------------------------ Python entry points
_dense_oracle = H.dense_tree_oracle  # pinned against the paged oracle in test_tree_oracle.py


def _paged_prefix(batch, hkv, d, cached, kv_dtype, seed, page=16):
    g = torch.Generator().manual_seed(seed)
    pages = (cached + page - 1) // page
    pool = batch * pages + 3
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    table = perm[: batch * pages].view(batch, pages).contiguous() if pages else torch.zeros(batch, 1, dtype=torch.int32)
    raw_k = torch.randn(pool, page, hkv, d, generator=g)
    raw_v = torch.randn(pool, page, hkv, d, generator=g)
    if kv_dtype == "fp8":
        import l20_pd_workloads as wl

        kc, ks = wl.quantize_fp8_e4m3(raw_k.to(torch.bfloat16))
        vc, vs = wl.quantize_fp8_e4m3(raw_v.to(torch.bfloat16))
        from oracle import paged_fp8_decode_ref as ref

        kf = ref.dequantize(kc.view(torch.uint8).numpy(), ks)
        vf = ref.dequantize(vc.view(torch.uint8).numpy(), vs)
    else:
        kc, vc, ks, vs = raw_k.to(kv_dtype), raw_v.to(kv_dtype), 1.0, 1.0
        kf, vf = kc.float().numpy(), vc.float().numpy()
    pk = np.stack([np.concatenate([kf[p] for p in table[i].tolist()], 0)[:cached] if pages else
                   np.zeros((0, hkv, d)) for i in range(batch)])
    pv = np.stack([np.concatenate([vf[p] for p in table[i].tolist()], 0)[:cached] if pages else
                   np.zeros((0, hkv, d)) for i in range(batch)])
    return kc.cuda(), vc.cuda(), ks, vs, table.cuda(), pk, pv


HYBRID = [
    # batch, hq, hkv, d, cached, draft, kv, page
    (2, 8, 2, 128, 1000, 4, "fp8", 16),
    (2, 28, 4, 128, 2049, 8, "fp8", 16),      # 56 columns -> two packed chunks
    (1, 8, 8, 128, 700, 40, torch.bfloat16, 16),  # 40 drafts (suffix > 32) -> chunks of 32
    (3, 16, 16, 64, 333, 5, torch.float16, 16),
    (2, 8, 2, 128, 0, 3, "fp8", 16),          # no cached prefix
    (2, 16, 4, 128, 1500, 6, "fp8", 32),      # 32-token pages
]


@pytest.mark.parametrize("case", HYBRID, ids=[f"h{i}" for i in range(len(HYBRID))])
def test_hybrid_tree_attention_paged_prefix(case):
    """Output against the pinned paged oracle (max-abs and cosine; drafts beyond a
    32-bit word against the dense restatement, pinned to it), and the prefix pass's
    LSE (what the path computes as LSE) against the oracle's prefix-only LSE."""
    import l20_tree_verify as tv

    batch, hq, hkv, d, cached, draft, kv, page = case
    print(f"hybrid {case}", flush=True)
    qdt = torch.bfloat16 if kv in ("fp8", torch.bfloat16) else torch.float16
    kc, vc, ks, vs, table, pk, pv = _paged_prefix(batch, hkv, d, cached, kv, seed=draft + cached, page=page)
    g = torch.Generator().manual_seed(99 + draft)
    query = torch.randn(batch, draft, hq, d, generator=g).to(qdt)
    sk = torch.randn(batch, draft, hkv, d, generator=g).to(qdt)
    sv = torch.randn(batch, draft, hkv, d, generator=g).to(qdt)
    mask = random_tree(draft, np.random.default_rng(draft))
    ws = tv.allocate_tree_attention_workspace(query.cuda())
    got = tv.hybrid_tree_attention_paged_prefix(
        query.cuda(), kc, vc, sk.cuda(), sv.cuda(), table, torch.from_numpy(mask).cuda(), cached,
        k_scale=ks, v_scale=vs, workspace=ws)
    torch.cuda.synchronize()
    assert got.shape == query.shape and got.dtype == qdt
    args = (query.float().numpy(), pk, pv, sk.float().numpy(), sv.float().numpy())
    if draft <= 32:
        exp, _ = H.paged_tree_oracle(*args, mask, d ** -0.5)
    else:
        exp = _dense_oracle(*args, mask, d ** -0.5)
    H.compare(got, None, exp, None, check_lse=False)
    # the prefix pass's LSE: every draft row over the cached keys alone
    p_lse = ws._buffers["prefix_lse"]
    padded = p_lse.shape[0] // batch
    got_lse = p_lse.view(batch, padded, hq)[:, :draft]
    _, exp_lse = H.paged_tree_oracle(*args, np.zeros((draft, draft), dtype=bool), d ** -0.5)
    if cached == 0:
        assert torch.isneginf(got_lse).all()
    else:
        err = np.abs(got_lse.cpu().numpy() - exp_lse) / np.maximum(1.0, np.abs(exp_lse))
        assert err.max() <= H.LSE_RTOL, float(err.max())


def test_hybrid_accepts_the_reference_tuple_workspace():
    """The reference's six-tensor workspace tuple is wrapped once and reused (its
    buffers persist), and anything else is refused."""
    import l20_tree_verify as tv

    batch, hq, hkv, d, cached, draft = 2, 8, 2, 128, 600, 5
    kc, vc, ks, vs, table, pk, pv = _paged_prefix(batch, hkv, d, cached, "fp8", seed=3)
    g = torch.Generator().manual_seed(4)
    query = torch.randn(batch, draft, hq, d, generator=g).to(torch.bfloat16).cuda()
    sk = torch.randn(batch, draft, hkv, d, generator=g).to(torch.bfloat16).cuda()
    sv = torch.randn(batch, draft, hkv, d, generator=g).to(torch.bfloat16).cuda()
    mask = torch.from_numpy(random_tree(draft, np.random.default_rng(5))).cuda()
    plain = tuple(tv.allocate_tree_attention_workspace(query))
    a = tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table, mask, cached, k_scale=ks, v_scale=vs,
                                              workspace=plain)
    wrapped = tv._as_workspace(plain, query)
    before = {k: v.data_ptr() for k, v in wrapped._buffers.items()}
    assert before, "the first call filled the wrapped workspace"
    b = tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table, mask, cached, k_scale=ks, v_scale=vs,
                                              workspace=plain)
    assert tv._as_workspace(plain, query)._buffers is wrapped._buffers
    assert {k: v.data_ptr() for k, v in wrapped._buffers.items()} == before
    assert torch.equal(a, b)
    with pytest.raises(TypeError):
        tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table, mask, cached, workspace=plain[:3])


def test_causal_verifier_equals_chain_hybrid_and_paged_tree():
    """causal_verifier_attention_paged == the hybrid path with the chain mask ==
    the in-cache tree path over the same keys (drafts appended as the newest
    tokens of 16-bit pages)."""
    import l20_tree_verify as tv

    batch, hq, hkv, d, cached, draft = 2, 16, 4, 128, 500, 6
    kc, vc, _, _, table, pk, pv = _paged_prefix(batch, hkv, d, cached, torch.bfloat16, seed=4)
    g = torch.Generator().manual_seed(5)
    query = torch.randn(batch, draft, hq, d, generator=g).to(torch.bfloat16).cuda()
    sk = torch.randn(batch, draft, hkv, d, generator=g).to(torch.bfloat16).cuda()
    sv = torch.randn(batch, draft, hkv, d, generator=g).to(torch.bfloat16).cuda()
    a = tv.causal_verifier_attention_paged(query, kc, vc, sk, sv, table, cached)
    b = tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table,
                                              tv.make_chain_tree_mask(draft, device="cuda"), cached)
    assert torch.equal(a, b)
    # in-cache layout: prefix + drafts in fresh pages of one cache
    total = cached + draft
    pages = (total + 15) // 16
    kfull = torch.zeros(batch * pages, 16, hkv, d, dtype=torch.bfloat16)
    vfull = torch.zeros_like(kfull)
    full_k = np.concatenate([pk, sk.float().cpu().numpy()], 1)
    full_v = np.concatenate([pv, sv.float().cpu().numpy()], 1)
    for i in range(batch):
        pad = np.zeros((pages * 16, hkv, d), dtype=np.float32)
        pad[:total] = full_k[i]
        kfull[i * pages:(i + 1) * pages] = torch.from_numpy(pad).view(pages, 16, hkv, d).to(torch.bfloat16)
        pad[:] = 0
        pad[:total] = full_v[i]
        vfull[i * pages:(i + 1) * pages] = torch.from_numpy(pad).view(pages, 16, hkv, d).to(torch.bfloat16)
    tbl = torch.arange(batch * pages, dtype=torch.int32).view(batch, pages).cuda()
    lens = torch.full((batch,), total, dtype=torch.int32).cuda()
    c = tv.paged_tree_verify_attention(query, kfull.cuda(), vfull.cuda(), tbl, lens,
                                       tv.make_chain_tree_mask(draft, device="cuda"))
    torch.cuda.synchronize()
    assert c.shape == query.shape
    assert (c.float() - a.float()).abs().max().item() <= H.OUT_ATOL


def test_paged_tree_verify_rejects_wide_tiles():
    import l20_tree_verify as tv

    q = torch.zeros(1, 8, 32, 128, dtype=torch.bfloat16, device="cuda")  # 8 drafts x group 8 = 64 columns
    kc = torch.zeros(4, 16, 4, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="32"):
        tv.paged_tree_verify_attention(q, kc, kc, torch.zeros(1, 4, dtype=torch.int32, device="cuda"),
                                       torch.full((1,), 40, dtype=torch.int32, device="cuda"),
                                       tv.make_chain_tree_mask(8, device="cuda"))


# ------------------------------------------------------------------ the fused suffix + merge kernel
@pytest.mark.parametrize("d,qdt,prefix_f32", [(128, torch.bfloat16, False), (64, torch.float16, True),
                                             (128, torch.float16, True)])
def test_tree_suffix_merge_c_abi_against_closed_form(d, qdt, prefix_f32):
    """out = (e^lse o_p + sum_j e^s_j v_j) / (e^lse + sum_j e^s_j) over the visible
    drafts, in float64; a row with an empty prefix (lse = -inf) and no visible
    draft is zero; 40 drafts exercise several key batches."""
    import l20_pd_cabi as cabi

    b, s, hq, hkv = 3, 40, 8, 2
    g = torch.Generator().manual_seed(d + s)
    q = torch.randn(b, s, hq, d, generator=g).to(qdt)
    sk = torch.randn(b, s, hkv, d, generator=g).to(qdt)
    sv = torch.randn(b, s, hkv, d, generator=g).to(qdt)
    mask = torch.from_numpy(random_tree(s, np.random.default_rng(3)))
    mask[5] = False                               # row 5 sees no draft
    po = torch.randn(b, s, hq, d, generator=g).to(torch.float32 if prefix_f32 else qdt)
    pl = torch.randn(b, s, hq, generator=g) * 3
    pl[1, 5, :] = float("-inf")                   # ... and, in sequence 1, no prefix either
    pl[2, :, 3] = float("-inf")                   # head 3 of sequence 2: suffix only
    scale = 0.3
    out = torch.empty(b, s, hq, d, dtype=qdt, device="cuda")
    t = [x.cuda() for x in (q, sk, sv, mask, po, pl)]
    args = cabi.tree_suffix_args_from_tensors(*t, out, scale)
    cabi.tree_suffix_merge(args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()

    qf, kf, vf = q.double().numpy(), sk.double().numpy(), sv.double().numpy()
    pof, plf, m = po.double().numpy(), pl.double().numpy(), mask.numpy()
    grp = hq // hkv
    exp = np.zeros((b, s, hq, d))
    for bi in range(b):
        for i in range(s):
            for h in range(hq):
                sc = kf[bi, :, h // grp] @ qf[bi, i, h] * scale
                w = np.where(m[i], np.exp(sc), 0.0)
                wp = np.exp(plf[bi, i, h])
                num = w @ vf[bi, :, h // grp] + (wp * pof[bi, i, h] if wp > 0 else 0.0)
                den = w.sum() + wp
                exp[bi, i, h] = num / den if den > 0 else 0.0
    got = out.double().cpu().numpy()
    assert np.array_equal(got[1, 5], np.zeros((hq, d)))
    # the 16-bit output's own rounding bounds the error (half an ulp: 2^-9 relative for
    # bf16, 2^-12 for fp16; twice that here), plus 1e-3 for fp32 arithmetic
    rel = 2.0 ** -8 if qdt == torch.bfloat16 else 2.0 ** -11
    assert np.all(np.abs(got - exp) <= rel * np.abs(exp) + 1e-3)


def _hybrid_inputs(batch, hq, hkv, d, cached, draft, seed, kv=torch.bfloat16):
    kc, vc, ks, vs, table, pk, pv = _paged_prefix(batch, hkv, d, cached, kv, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    qdt = torch.bfloat16 if kv in ("fp8", torch.bfloat16) else torch.float16
    query = torch.randn(batch, draft, hq, d, generator=g).to(qdt).cuda()
    sk = torch.randn(batch, draft, hkv, d, generator=g).to(qdt).cuda()
    sv = torch.randn(batch, draft, hkv, d, generator=g).to(qdt).cuda()
    mask = torch.from_numpy(random_tree(draft, np.random.default_rng(seed))).cuda()
    return dict(query=query, kc=kc, vc=vc, ks=ks, vs=vs, table=table, sk=sk, sv=sv, mask=mask, pk=pk, pv=pv)


@pytest.mark.parametrize("draft,hq,hkv", [(8, 28, 4), (5, 8, 2)])  # two packed chunks; one padded chunk
def test_hybrid_warmed_workspace_allocates_nothing_and_replays_in_a_graph(draft, hq, hkv):
    import l20_tree_verify as tv

    x = _hybrid_inputs(2, hq, hkv, 128, 1500, draft, seed=draft, kv="fp8")
    ws = tv.allocate_tree_attention_workspace(x["query"])
    out = torch.empty_like(x["query"])

    def call():
        return tv.hybrid_tree_attention_paged_prefix(
            x["query"], x["kc"], x["vc"], x["sk"], x["sv"], x["table"], x["mask"], 1500,
            workspace=ws, k_scale=x["ks"], v_scale=x["vs"], output=out)

    call()
    torch.cuda.synchronize()
    first = out.clone()
    exp = _dense_oracle(x["query"].float().cpu().numpy(), x["pk"], x["pv"], x["sk"].float().cpu().numpy(),
                        x["sv"].float().cpu().numpy(), x["mask"].cpu().numpy(), 128 ** -0.5)
    assert np.abs(first.float().cpu().numpy() - exp).max() <= H.OUT_ATOL
    before = torch.cuda.memory_stats()["allocation.all.allocated"]
    call()
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == before, "a warmed call allocated"
    assert torch.equal(out, first)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.synchronize()
    q0 = x["query"].clone()
    for r in range(3):
        # new draft queries in place, then a replay against an eager call on them
        x["query"].copy_(q0 * (1.0 + 0.25 * r))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        call()
        torch.cuda.synchronize()
        assert torch.equal(replayed, out), r


def test_hybrid_contiguous_pages_equal_block_table():
    import l20_tree_verify as tv

    batch, hq, hkv, d, cached, draft = 3, 16, 4, 128, 700, 6
    pages = (cached + 15) // 16
    g = torch.Generator().manual_seed(8)
    base = torch.tensor([5, 5 + pages + 2, 5 + 2 * pages + 9], dtype=torch.int32)
    pool = int(base.max()) + pages + 1
    kc = torch.randn(pool, 16, hkv, d, generator=g).to(torch.bfloat16).cuda()
    vc = torch.randn(pool, 16, hkv, d, generator=g).to(torch.bfloat16).cuda()
    table = (base[:, None] + torch.arange(pages, dtype=torch.int32)[None, :]).cuda()
    query = torch.randn(batch, draft, hq, d, generator=g).to(torch.bfloat16).cuda()
    sk = torch.randn(batch, draft, hkv, d, generator=g).to(torch.bfloat16).cuda()
    sv = torch.randn(batch, draft, hkv, d, generator=g).to(torch.bfloat16).cuda()
    mask = torch.from_numpy(random_tree(draft, np.random.default_rng(1))).cuda()
    a = tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table, mask, cached)
    junk = torch.full_like(table, -1)  # ignored with contiguous pages
    b = tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, junk, mask, cached,
                                              contiguous_pages=True, page_base=base.cuda(), block_t=128)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="block_t"):
        tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table, mask, cached, block_t=48)
    with pytest.raises(ValueError, match="page_base"):
        tv.hybrid_tree_attention_paged_prefix(query, kc, vc, sk, sv, table, mask, cached, contiguous_pages=True)


def test_dispatch_helpers_route_to_the_hybrid_and_causal_paths(monkeypatch):
    import l20_tree_attention_dispatch as disp
    import l20_tree_verify as tv

    x = _hybrid_inputs(2, 16, 4, 128, 4100, 6, seed=17)
    args = (x["query"], x["kc"], x["vc"], x["sk"], x["sv"], x["table"])
    monkeypatch.delenv(disp.ENABLE_ENV, raising=False)
    assert disp.maybe_l20_tree_attention(*args, x["mask"], 4100) is None
    monkeypatch.setenv(disp.ENABLE_ENV, "1")
    got = disp.maybe_l20_tree_attention(*args, x["mask"], 4100)
    want = tv.hybrid_tree_attention_paged_prefix(*args, x["mask"], 4100)
    torch.cuda.synchronize()
    assert got is not None and torch.equal(got, want)
    got_c = disp.maybe_l20_causal_verifier_attention(*args, 4100)
    want_c = tv.causal_verifier_attention_paged(*args, 4100)
    torch.cuda.synchronize()
    assert got_c is not None and torch.equal(got_c, want_c)
    assert disp.maybe_l20_tree_attention(*args, x["mask"], 1000) is None  # below the threshold


CONTIG = [
    # batch, hq, hkv, d, cached, draft, dtype, layout
    (2, 16, 4, 128, 1020, 4, torch.bfloat16, "contiguous"),   # T = 1024: pages are a view
    (2, 28, 4, 128, 777, 8, torch.bfloat16, "contiguous"),    # T % 16 != 0: copied into pages
    (3, 8, 8, 64, 300, 5, torch.float16, "strided"),          # a slice of a wider tensor: copied
    (1, 8, 2, 128, 0, 3, torch.bfloat16, "contiguous"),       # no cached prefix
]


@pytest.mark.parametrize("case", CONTIG, ids=[f"c{i}" for i in range(len(CONTIG))])
def test_contiguous_cache_tree_attention(case):
    """hybrid_tree_attention / hybrid_tree_attention_split (the reference's contiguous-cache
    entry points, triton_tree_attention.py:706-886) against the pinned paged oracle
    (max-abs and cosine)."""
    import l20_tree_verify as tv

    batch, hq, hkv, d, cached, draft, dtype, layout = case
    total = cached + draft
    g = torch.Generator().manual_seed(cached + draft)
    query = torch.randn(batch, draft, hq, d, generator=g).to(dtype)
    if layout == "strided":
        wide_k = torch.randn(batch, total, hkv, 2 * d, generator=g).to(dtype)
        wide_v = torch.randn(batch, total, hkv, 2 * d, generator=g).to(dtype)
        key, value = wide_k.cuda()[..., :d], wide_v.cuda()[..., :d]
        assert not key.is_contiguous()
    else:
        key = torch.randn(batch, total, hkv, d, generator=g).to(dtype).cuda()
        value = torch.randn(batch, total, hkv, d, generator=g).to(dtype).cuda()
    mask = torch.from_numpy(random_tree(draft, np.random.default_rng(draft)))
    kf, vf = key.float().cpu().numpy(), value.float().cpu().numpy()
    exp, _ = H.paged_tree_oracle(query.float().numpy(), kf[:, :cached], vf[:, :cached], kf[:, cached:],
                                 vf[:, cached:], mask.numpy(), d ** -0.5)
    a = tv.hybrid_tree_attention(query.cuda(), key, value, mask.cuda(), cached)
    ws = tv.allocate_tree_attention_workspace(query.cuda())
    b = tv.hybrid_tree_attention_split(query.cuda(), key, value, mask.cuda(), cached, workspace=ws, block_t=64)
    b2 = tv.hybrid_tree_attention_split(query.cuda(), key, value, mask.cuda(), cached, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(b, b2)
    H.compare(a, None, exp, None, check_lse=False)
    with pytest.raises(ValueError, match="cached_length"):
        tv.hybrid_tree_attention(query.cuda(), key, value, mask.cuda(), cached + 1)
