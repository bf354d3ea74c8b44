"""Pins for the CPU oracle (oracle/paged_fp8_decode_ref.py), CPU only.

Each oracle function is checked against something other than its own formula:
torch's float8_e4m3fn conversion (a library routine), closed forms, the
reference's masked-attention known answer, an independent float64 loop, and
invariances.  The mutation tests at the end plant plausible mistakes in a copy
of the oracle and show that the checks here catch them.
"""

import math

import numpy as np
import pytest
import torch

from oracle import paged_fp8_decode_ref as ref


# ---------------------------------------------------------------- fp8 codec
def test_decode_table_matches_closed_form_and_torch():
    table = ref.e4m3fn_decode_table()
    codes = torch.arange(256, dtype=torch.uint8)
    via_torch = codes.view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(table)
    assert np.array_equal(np.flatnonzero(nan), [0x7F, 0xFF])
    assert np.array_equal(np.isnan(via_torch), nan)
    assert np.array_equal(table[~nan], via_torch[~nan])
    # spot values of the OCP e4m3fn format
    assert table[0x00] == 0.0 and table[0x80] == 0.0 and np.signbit(table[0x80])
    assert table[0x01] == 2.0 ** -9          # smallest subnormal
    assert table[0x08] == 2.0 ** -6          # smallest normal
    assert table[0x38] == 1.0
    assert table[0x7E] == 448.0 and table[0xFE] == -448.0


def test_encode_matches_torch_rne_on_random_and_midpoints():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 50,
        rng.uniform(-448, 448, 20000).astype(np.float32),
        rng.standard_normal(5000).astype(np.float32) * 1e-3,
    ])
    pos = ref.e4m3fn_decode_table()[:0x7F].astype(np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    mids = mids[(mids.astype(np.float64) == (pos[1:] + pos[:-1]) / 2)]  # exact midpoints only
    vals = np.concatenate([vals, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1000)])
    vals = np.clip(vals, -448, 448)
    ours = ref.encode_e4m3fn(vals)
    theirs = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # -0.0 vs +0.0 for values rounding to zero: compare decoded values and sign
    assert np.array_equal(ref.e4m3fn_to_f32(ours), ref.e4m3fn_to_f32(theirs))
    assert np.array_equal(ours, theirs)


def test_quantize_matches_torch_workload_quantizer():
    import l20_pd_workloads as wl

    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 16, 3, 64, generator=g).to(torch.bfloat16)
    codes_t, scale_t = wl.quantize_fp8_e4m3(x)
    codes_n, scale_n = ref.quantize_fp8_e4m3(x.float().numpy())
    assert np.float32(scale_t) == np.float32(scale_n)
    assert np.array_equal(codes_t.view(torch.uint8).numpy(), codes_n)
    codes_t, scales_t = wl.quantize_fp8_e4m3(x, per_head_axis=2)
    codes_n, scales_n = ref.quantize_fp8_e4m3_per_head(x.float().numpy(), head_axis=2)
    assert np.array_equal(scales_t.numpy(), scales_n)
    assert np.array_equal(codes_t.view(torch.uint8).numpy(), codes_n)


def test_e5m2_decode_table_matches_torch_and_fp16_top_byte():
    table = ref.e5m2_decode_table()
    codes = torch.arange(256, dtype=torch.uint8)
    via_torch = codes.view(torch.float8_e5m2).float().numpy()
    # e5m2 is fp16 with the low 8 mantissa bits dropped
    via_fp16 = (codes.to(torch.int16) << 8).view(torch.float16).float().numpy()
    nan = np.isnan(table)
    assert np.array_equal(np.flatnonzero(nan), [0x7D, 0x7E, 0x7F, 0xFD, 0xFE, 0xFF])
    for other in (via_torch, via_fp16):
        assert np.array_equal(np.isnan(other), nan)
        assert np.array_equal(table[~nan], other[~nan])
        assert np.array_equal(np.signbit(table[~nan]), np.signbit(other[~nan]))
    assert table[0x7C] == np.inf and table[0xFC] == -np.inf
    assert table[0x01] == 2.0 ** -16 and table[0x04] == 2.0 ** -14 and table[0x3C] == 1.0
    assert table[0x7B] == 57344.0
    assert np.array_equal(ref.fp8_to_f32(np.array([0x3C, 0xBC]), "e5m2"), [1.0, -1.0])
    with pytest.raises(ValueError):
        ref.decode_table("e4m3fnuz")


def _e5m2_case(seed, batch, hq, hkv, d, lens, q_len=1):
    """make_case's layout with e5m2 codes (via torch's float8_e5m2 rounding)."""
    case = make_case(seed, batch, hq, hkv, d, lens, q_len=q_len)
    rng = np.random.default_rng(seed + 100)
    for name in ("key_cache", "value_cache"):
        raw = torch.from_numpy(rng.standard_normal(case[name].shape).astype(np.float32) * 300)
        case[name] = raw.to(torch.float8_e5m2).view(torch.uint8).numpy()
    case["k_scale"], case["v_scale"] = 0.01, 0.003
    return case


@pytest.mark.parametrize("spec", [dict(seed=5, batch=2, hq=4, hkv=2, d=64, lens=[17, 33]),
                                  dict(seed=6, batch=2, hq=4, hkv=2, d=64, lens=[21, 9], q_len=4)])
def test_e5m2_reference_matches_brute_force_and_split(spec):
    case = _e5m2_case(**spec)
    out, lse = run(ref.reference, case, kv_format="e5m2")
    out64, lse64 = run(ref.brute_force_fp64, case, kv_format="e5m2")
    np.testing.assert_allclose(out, out64, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, lse64, atol=2e-6, rtol=1e-6)
    out_s, lse_s = run(ref.split_reference, case, split_size=16, kv_format="e5m2")
    np.testing.assert_allclose(out_s, out64, atol=1e-5)
    np.testing.assert_allclose(lse_s, lse64, atol=1e-5)
    # the same bytes read as e4m3fn give a different answer: the format switch is live
    out_wrong, _ = run(ref.reference, case)
    assert not np.allclose(out_wrong, out, atol=1e-3, equal_nan=True)


# ---------------------------------------------------------------- helpers
def make_case(seed, batch, hq, hkv, d, lens, q_len=1, per_head=False, pool_extra=3):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    pages_per = (lens + 15) // 16
    pool = int(pages_per.sum()) + pool_extra
    perm = rng.permutation(pool)
    table = np.zeros((batch, max(1, int(pages_per.max()))), dtype=np.int32)
    off = 0
    for b in range(batch):
        table[b, :pages_per[b]] = perm[off:off + pages_per[b]]
        off += pages_per[b]
    query = rng.standard_normal((batch * q_len, hq, d)).astype(np.float32)
    k = rng.standard_normal((pool, 16, hkv, d)).astype(np.float32)
    v = rng.standard_normal((pool, 16, hkv, d)).astype(np.float32)
    if per_head:
        kc, ks = ref.quantize_fp8_e4m3_per_head(k)
        vc, vs = ref.quantize_fp8_e4m3_per_head(v)
    else:
        kc, ks = ref.quantize_fp8_e4m3(k)
        vc, vs = ref.quantize_fp8_e4m3(v)
    return dict(query=query, key_cache=kc, value_cache=vc, block_table=table, seq_lens=lens,
                k_scale=ks, v_scale=vs, q_len=q_len)


def run(fn, case, **kw):
    c = dict(case)
    q_len = c.pop("q_len")
    return fn(c["query"], c["key_cache"], c["value_cache"], c["block_table"], c["seq_lens"],
              c["k_scale"], c["v_scale"], q_len=q_len, **kw)


TINY = [
    dict(seed=1, batch=2, hq=4, hkv=2, d=64, lens=[17, 33]),
    dict(seed=2, batch=1, hq=3, hkv=1, d=128, lens=[40], per_head=False),
    dict(seed=3, batch=2, hq=4, hkv=2, d=64, lens=[21, 9], q_len=4, per_head=True),
    dict(seed=4, batch=1, hq=2, hkv=2, d=64, lens=[16], q_len=2),
]


@pytest.mark.parametrize("spec", TINY)
def test_reference_matches_fp64_brute_force(spec):
    case = make_case(**spec)
    out, lse = run(ref.reference, case)
    out64, lse64 = run(ref.brute_force_fp64, case)
    np.testing.assert_allclose(out, out64, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, lse64, atol=2e-6, rtol=1e-6)


@pytest.mark.parametrize("spec", TINY)
@pytest.mark.parametrize("split", [16, 32, 48])
def test_split_reference_matches_reference(spec, split):
    case = make_case(**spec)
    out, lse = run(ref.reference, case, acc_dtype=np.float64)
    out_s, lse_s = run(ref.split_reference, case, split_size=split)
    np.testing.assert_allclose(out_s, out, atol=1e-6)
    np.testing.assert_allclose(lse_s, lse, atol=1e-6)


# ---------------------------------------------------------------- closed forms
def _identity_case(d=64, length=48, hkv=1, hq=2):
    pages = (length + 15) // 16
    table = np.arange(pages, dtype=np.int32)[None]
    return table, np.array([length], dtype=np.int32), pages


def test_equal_keys_give_mean_of_values_and_lse_s_plus_log_l():
    d, length = 64, 48
    table, lens, pages = _identity_case(d, length)
    rng = np.random.default_rng(7)
    kc = np.full((pages, 16, 1, d), 0x38, dtype=np.uint8)           # every key element = 1.0
    vc = ref.encode_e4m3fn(np.clip(rng.standard_normal((pages, 16, 1, d)) * 4, -448, 448)).reshape(pages, 16, 1, d)
    q = rng.standard_normal((1, 2, d)).astype(np.float32)
    out, lse = ref.reference(q, kc, vc, table, lens, 1.0, 0.5)
    vals = ref.e4m3fn_to_f32(vc).reshape(-1, d)[:length] * 0.5
    np.testing.assert_allclose(out[0, 0], vals.mean(axis=0), atol=1e-6)
    s = q[0].sum(axis=1) * d ** -0.5                                 # q . 1 * scale
    np.testing.assert_allclose(lse[0], s + math.log(length), rtol=1e-6)


def test_single_token_returns_v0_and_dominant_score_selects_its_row():
    d = 128
    table, lens, pages = _identity_case(d, 1)
    rng = np.random.default_rng(8)
    kc = ref.encode_e4m3fn(np.clip(rng.standard_normal((pages, 16, 1, d)), -448, 448))
    vc = ref.encode_e4m3fn(np.clip(rng.standard_normal((pages, 16, 1, d)), -448, 448))
    q = rng.standard_normal((1, 1, d)).astype(np.float32)
    out, _ = ref.reference(q, kc, vc, table, lens, 1.0, 2.0)
    np.testing.assert_allclose(out[0, 0], ref.e4m3fn_to_f32(vc[0, 0, 0]) * 2.0, rtol=1e-6)
    # one key aligned with a large query dominates the softmax
    table, lens, pages = _identity_case(d, 32)
    kc = np.zeros((pages, 16, 1, d), dtype=np.uint8)
    kc[1, 3, 0, :] = 0x7E                                           # token 19 = 448 everywhere
    q = np.ones((1, 1, d), dtype=np.float32)
    vc = ref.encode_e4m3fn(np.clip(rng.standard_normal((pages, 16, 1, d)), -448, 448))
    out, _ = ref.reference(q, kc, vc, table, lens, 1.0, 1.0)
    np.testing.assert_allclose(out[0, 0], ref.e4m3fn_to_f32(vc[1, 3, 0]), rtol=1e-6)


def _as_pages(case, page):
    """The same logical tokens in ``page``-token pages: 16-token page ``j`` of a
    sequence goes to row ``16 (j % m)`` of page ``table[b, j // m]`` (m = page / 16)
    of a pool laid out afresh, with a permuted page order."""
    m = page // 16
    table16, kc16, vc16 = case["block_table"], case["key_cache"], case["value_cache"]
    batch, n16 = table16.shape
    n_p = (n16 + m - 1) // m
    rng = np.random.default_rng(page)
    perm = rng.permutation(batch * n_p + 2)
    table = perm[:batch * n_p].reshape(batch, n_p).astype(np.int32)
    shape = (batch * n_p + 2, page) + kc16.shape[2:]
    kc = np.zeros(shape, dtype=kc16.dtype)
    vc = np.zeros(shape, dtype=vc16.dtype)
    for b in range(batch):
        for j in range(n16):
            kc[table[b, j // m], 16 * (j % m):16 * (j % m) + 16] = kc16[table16[b, j]]
            vc[table[b, j // m], 16 * (j % m):16 * (j % m) + 16] = vc16[table16[b, j]]
    return dict(case, key_cache=kc, value_cache=vc, block_table=table)


@pytest.mark.parametrize("page", [32, 64, 48])
@pytest.mark.parametrize("spec", [dict(seed=11, batch=2, hq=4, hkv=2, d=64, lens=[70, 33]),
                                  dict(seed=12, batch=2, hq=4, hkv=2, d=64, lens=[45, 96], q_len=3)])
def test_pages_of_any_multiple_of_16_tokens(spec, page):
    """Pages of P tokens (the reference hook's ``token // page_size``, ``token %
    page_size`` gather, integrations/vllm/l20_paged_split_kv.py:182-200): the same
    logical tokens give bitwise the 16-token-page answer, and the fp64 loop agrees."""
    case16 = make_case(**spec)
    case = _as_pages(case16, page)
    out, lse = run(ref.reference, case)
    out16, lse16 = run(ref.reference, case16)
    assert np.array_equal(out, out16) and np.array_equal(lse, lse16)
    out64, lse64 = run(ref.brute_force_fp64, case)
    np.testing.assert_allclose(out, out64, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, lse64, atol=2e-6, rtol=1e-6)
    # The kernels' view: the cache as 16-token sub-pages, tile j of a sequence at
    # sub-page table[b, j // m] * m + j % m -- bitwise the same answer; without the
    # sub-page term it reads other tokens.
    m = page // 16
    sub = dict(case, key_cache=case["key_cache"].reshape((-1, 16) + case["key_cache"].shape[2:]),
               value_cache=case["value_cache"].reshape((-1, 16) + case["value_cache"].shape[2:]))
    j = np.arange(case["block_table"].shape[1] * m)
    out_sub, lse_sub = run(ref.reference, dict(sub, block_table=case["block_table"][:, j // m] * m + j % m))
    assert np.array_equal(out_sub, out) and np.array_equal(lse_sub, lse)
    out_wrong, _ = run(ref.reference, dict(sub, block_table=case["block_table"][:, j // m] * m))
    assert not np.allclose(out_wrong, out, atol=1e-3)


def test_reference_masked_attention_known_answer():
    """tests/test_tree_attention.py:36-53 of the reference, restated for the chain mask.

    Two draft rows over 2 cached + 2 draft keys; query = ones(2), keys
    [1,0],[0,1],[2,0],[0,2], values 1,2,4,8 in dim 0, scale 2^-0.5.  With the
    causal chain, row 0 sees keys 0..2 and row 1 sees keys 0..3.
    """
    d = 64  # pad the 2-dim example with zeros (no effect on scores or values)
    k = np.zeros((1, 16, 1, d), dtype=np.float32)
    v = np.zeros((1, 16, 1, d), dtype=np.float32)
    k[0, 0, 0, 0], k[0, 1, 0, 1], k[0, 2, 0, 0], k[0, 3, 0, 1] = 1, 1, 2, 2
    v[0, :4, 0, 0] = [1, 2, 4, 8]
    kc, vc = ref.encode_e4m3fn(k), ref.encode_e4m3fn(v)
    q = np.zeros((2, 1, d), dtype=np.float32)
    q[:, 0, :2] = 1.0
    out, _ = ref.reference(q, kc, vc, np.array([[0]], np.int32), np.array([4], np.int32), 1.0, 1.0,
                           softmax_scale=2 ** -0.5, q_len=2)
    a, b2 = math.exp(2 ** -0.5), math.exp(2 * 2 ** -0.5)
    row0 = (1 * a + 2 * a + 4 * b2) / (a + a + b2)
    row1 = (1 * a + 2 * a + 4 * b2 + 8 * b2) / (a + a + b2 + b2)
    np.testing.assert_allclose(out[:, 0, 0], [row0, row1], rtol=1e-6)


# ---------------------------------------------------------------- invariances
def test_page_permutation_invariance():
    case = make_case(11, 2, 4, 2, 64, [70, 35], pool_extra=10)
    out, lse = run(ref.reference, case)
    # move every page to a new physical slot
    rng = np.random.default_rng(12)
    pool = case["key_cache"].shape[0]
    perm = rng.permutation(pool)
    inv = np.argsort(perm)
    moved = dict(case, key_cache=case["key_cache"][inv], value_cache=case["value_cache"][inv],
                 block_table=perm[case["block_table"]].astype(np.int32))
    out2, lse2 = run(ref.reference, moved)
    np.testing.assert_array_equal(out, out2)
    np.testing.assert_array_equal(lse, lse2)


def test_gqa_equals_mha_with_replicated_heads():
    case = make_case(13, 2, 6, 2, 64, [30, 50])
    out, lse = run(ref.reference, case)
    mha = dict(case, key_cache=np.repeat(case["key_cache"], 3, axis=2),
               value_cache=np.repeat(case["value_cache"], 3, axis=2))
    out2, lse2 = run(ref.reference, mha)
    np.testing.assert_allclose(out, out2, atol=1e-6)
    np.testing.assert_allclose(lse, lse2, atol=1e-6)


def test_equal_per_head_scales_equal_per_tensor():
    case = make_case(14, 1, 4, 2, 64, [45])
    out, lse = run(ref.reference, case)
    ph = dict(case, k_scale=np.full(2, case["k_scale"], np.float32), v_scale=np.full(2, case["v_scale"], np.float32))
    out2, lse2 = run(ref.reference, ph)
    np.testing.assert_array_equal(out, out2)
    np.testing.assert_array_equal(lse, lse2)


def test_causal_row_equals_single_query_on_shortened_sequence():
    q_len = 4
    case = make_case(15, 2, 4, 2, 64, [37, 20], q_len=q_len)
    out, lse = run(ref.reference, case)
    for i in range(q_len):
        rows = np.arange(2) * q_len + i
        single = dict(case, query=case["query"][rows], q_len=1,
                      seq_lens=case["seq_lens"] - (q_len - 1 - i))
        o1, l1 = run(ref.reference, single)
        np.testing.assert_allclose(out[rows], o1, atol=1e-6)
        np.testing.assert_allclose(lse[rows], l1, atol=1e-6)


def test_empty_rows_give_zero_and_minus_inf():
    case = make_case(16, 2, 2, 1, 64, [0, 2], q_len=3)
    out, lse = run(ref.reference, case)
    assert np.all(out[:3] == 0) and np.all(np.isneginf(lse[:3]))     # L = 0
    assert np.all(out[3] == 0) and np.all(np.isneginf(lse[3]))       # row 0 of L=2 sees nothing
    assert np.all(np.isfinite(lse[4:]))
    out64, lse64 = run(ref.brute_force_fp64, case)
    np.testing.assert_allclose(out, out64, atol=2e-6)


# ---------------------------------------------------------------- planted mistakes
def _mutant(kind):
    """A copy of ``ref.reference`` with one plausible bug planted."""

    def mutant(query, key_cache, value_cache, block_table, seq_lens, k_scale, v_scale, *, q_len=1, **kw):
        if kind == "causal_off_by_one":
            seq_lens = np.asarray(seq_lens) - 1
            out, lse = ref.reference(query, key_cache, value_cache, block_table, seq_lens, k_scale, v_scale,
                                     q_len=q_len, **kw)
            return out, lse
        if kind == "head_modulo":   # kv head = h % Hkv instead of h // G
            hkv = key_cache.shape[2]
            g = query.shape[1] // hkv
            order = np.array([(h % hkv) * g + h // hkv for h in range(query.shape[1])])
            out, lse = ref.reference(query[:, order], key_cache, value_cache, block_table, seq_lens, k_scale,
                                     v_scale, q_len=q_len, **kw)
            inv = np.argsort(order)
            return out[:, inv], lse[:, inv]
        if kind == "no_v_scale":
            return ref.reference(query, key_cache, value_cache, block_table, seq_lens, k_scale, 1.0,
                                 q_len=q_len, **kw)
        if kind == "page_slot_swapped":  # token -> (t % 16, t // 16)
            kc = np.swapaxes(key_cache, 0, 1).copy() if key_cache.shape[0] == 16 else key_cache[:, ::-1]
            vc = np.swapaxes(value_cache, 0, 1).copy() if value_cache.shape[0] == 16 else value_cache[:, ::-1]
            return ref.reference(query, kc, vc, block_table, seq_lens, k_scale, v_scale, q_len=q_len, **kw)
        raise ValueError(kind)

    return mutant


@pytest.mark.parametrize("kind", ["causal_off_by_one", "head_modulo", "no_v_scale", "page_slot_swapped"])
def test_planted_mistakes_are_caught_by_brute_force(kind):
    case = make_case(21, 2, 4, 2, 64, [23, 31], q_len=2)
    if kind == "no_v_scale":
        case["v_scale"] = 0.37
    good, _ = run(ref.brute_force_fp64, case)
    bad, _ = run(_mutant(kind), case)
    assert not np.allclose(bad, good, atol=1e-3)


# ------------------------------------------------------------ CSR page lists, 16-bit KV siblings
def _to_csr(table, lens, rng=None, pad=0):
    """The reference benchmark's CSR form (``benchmark_cuda_paged_decode.py:67-73``):
    ``page_indices`` = the used pages of each row, ``page_indptr`` = row offsets.
    ``pad`` extra garbage entries between rows check that offsets, not row lengths, are used."""
    rows, indptr = [], [0]
    for b, L in enumerate(lens):
        n = (int(L) + 15) // 16
        rows.append(np.asarray(table[b, :n], dtype=np.int32))
        if pad:
            rows.append(np.full(pad, 10**6, dtype=np.int32))
        indptr.append(indptr[-1] + n + pad)
    return np.concatenate(rows) if rows else np.zeros(0, np.int32), np.asarray(indptr, dtype=np.int32)


@pytest.mark.parametrize("spec", TINY[:3])
def test_csr_page_list_equals_block_table(spec):
    case = make_case(**spec)
    exp = run(ref.reference, case)
    for pad in (0, 3):
        indices, indptr = _to_csr(case["block_table"], case["seq_lens"], pad=pad)
        c = dict(case, block_table=indices)
        got = run(ref.reference, c, page_indptr=indptr)
        np.testing.assert_array_equal(got[0], exp[0])
        np.testing.assert_array_equal(got[1], exp[1])


def test_csr_with_shifted_offsets_is_caught():
    """A planted off-by-one row offset (indptr[b + 1] for indptr[b]) must change the result."""
    case = make_case(seed=9, batch=3, hq=4, hkv=2, d=64, lens=[40, 36, 33])  # 3 pages each
    indices, indptr = _to_csr(case["block_table"], case["seq_lens"])
    good = run(ref.reference, dict(case, block_table=indices), page_indptr=indptr)
    shifted = np.concatenate([indptr[1:], indptr[-1:] + 3])
    indices_padded = np.concatenate([indices, np.zeros(8, np.int32)])
    bad = run(ref.reference, dict(case, block_table=indices_padded), page_indptr=shifted)
    assert not np.allclose(good[0], bad[0])


def test_dense_kv_reference_equals_fp8_path_on_representable_values():
    """16-bit caches holding exactly the dequantised fp8 values (scale 1) reproduce the
    fp8 oracle bit for bit; the fp8 oracle itself is pinned by the fp64 brute force."""
    case = make_case(seed=12, batch=2, hq=8, hkv=2, d=128, lens=[70, 33], q_len=2)
    k = ref.e4m3fn_to_f32(case["key_cache"])
    v = ref.e4m3fn_to_f32(case["value_cache"])
    exp = ref.reference(case["query"], case["key_cache"], case["value_cache"], case["block_table"],
                        case["seq_lens"], 1.0, 1.0, q_len=2)
    got = ref.reference_dense_kv(case["query"], k, v, case["block_table"], case["seq_lens"], q_len=2)
    np.testing.assert_array_equal(got[0], exp[0])
    np.testing.assert_array_equal(got[1], exp[1])
    bf = ref.brute_force_fp64(case["query"], case["key_cache"], case["value_cache"], case["block_table"],
                              case["seq_lens"], 1.0, 1.0, q_len=2)
    np.testing.assert_allclose(got[0], bf[0], rtol=2e-5, atol=1e-3)  # values up to 448


def test_dense_kv_single_token_and_equal_keys_closed_forms():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, 64)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, 1, 64)), 16, axis=1).astype(np.float32)  # 16 equal keys
    v = rng.standard_normal((1, 16, 1, 64)).astype(np.float32)
    table = np.zeros((1, 1), np.int32)
    out, lse = ref.reference_dense_kv(q, k, v, table, np.array([1]))
    np.testing.assert_allclose(out[0], np.broadcast_to(v[0, 0, 0], (2, 64)), rtol=1e-6)
    out, lse = ref.reference_dense_kv(q, k, v, table, np.array([16]))
    np.testing.assert_allclose(out[0], np.broadcast_to(v[0, :, 0].mean(0), (2, 64)), rtol=1e-5, atol=1e-6)
    s = (q[0] @ k[0, 0, 0]) / 8.0
    np.testing.assert_allclose(lse[0], s + math.log(16), rtol=1e-5)


# ------------------------------------------------------------ tree (ancestor-mask) verify
def test_reference_tree_attention_known_answer():
    """The reference's KAT with its irregular ancestor mask (tests/test_tree_attention.py:36-53):
    2 cached + 2 draft tokens, mask [[T, F], [F, T]], all-ones query, D=2."""
    q = np.ones((2, 1, 2), np.float32)
    k = np.array([[1, 0], [0, 1], [2, 0], [0, 2]], np.float32).reshape(4, 1, 1, 2)
    v = np.array([[1, 0], [2, 0], [4, 0], [8, 0]], np.float32).reshape(4, 1, 1, 2)
    kc = np.zeros((1, 16, 1, 2), np.float32)
    vc = np.zeros_like(kc)
    kc[0, :4], vc[0, :4] = k[:, 0], v[:, 0]
    bits = ref.tree_bits_from_mask(np.array([[True, False], [False, True]]))
    assert bits.tolist() == [1, 2]
    out, _ = ref.reference_dense_kv(q, kc, vc, np.zeros((1, 1), np.int32), np.array([4]), q_len=2, tree_mask=bits)
    s = 2 ** -0.5
    for row, visible in enumerate(([0, 1, 2], [0, 1, 3])):
        scores = np.array([k[t, 0, 0].sum() * s for t in visible])
        p = np.exp(scores - scores.max())
        p /= p.sum()
        want = (p[:, None] * v[visible, 0, 0]).sum(0)
        np.testing.assert_allclose(out[row, 0], want, rtol=1e-6)


def test_chain_tree_mask_equals_causal_rule():
    case = make_case(seed=21, batch=2, hq=4, hkv=2, d=64, lens=[21, 9], q_len=4, per_head=True)
    chain = ref.tree_bits_from_mask(np.tril(np.ones((4, 4), bool)))
    a = run(ref.reference, case)
    b = run(ref.reference, case, tree_mask=chain)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_tree_reference_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    q_len = 5
    case = make_case(seed=30 + seed, batch=2, hq=4, hkv=2, d=64, lens=[37, 12], q_len=q_len)
    # random trees: each draft token's parent is an earlier draft token (or the prefix)
    masks = []
    for _ in range(2):
        anc = np.zeros((q_len, q_len), bool)
        for i in range(q_len):
            anc[i, i] = True
            parent = rng.integers(-1, i) if i else -1
            if parent >= 0:
                anc[i] |= anc[parent]
        masks.append(anc)
    bits = ref.tree_bits_from_mask(np.stack(masks))
    got = run(ref.reference, case, tree_mask=bits)
    want = run(ref.brute_force_fp64, case, tree_mask=bits)
    np.testing.assert_allclose(got[0], want[0], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(got[1], want[1], rtol=2e-5, atol=2e-6)
    # a planted mistake (bits shifted by one draft position) is caught
    bad = run(ref.reference, case, tree_mask=bits << 1)
    assert not np.allclose(bad[0], want[0], atol=1e-3)


# ---------------------------------------------------------------- literal fp16 dequantisation
# The reference oracle rounds the dequantised K/V to fp16 before attending
# (scripts/smoke_cuda_paged_fp8_decode_op.py:23-24); this oracle keeps fp32.
def _power_of_two_case():
    case = make_case(seed=21, batch=2, hq=4, hkv=2, d=64, lens=[37, 70], q_len=2)
    return dict(case, k_scale=0.125, v_scale=2.0 ** -5)


@pytest.mark.parametrize("spec", TINY)
def test_acc_f64_is_closer_to_brute_force_than_acc_f32(spec):
    """float64 accumulation (outputs still stored as float32, K/V dequantised
    in float32 as the reference does) lands nearer the float64 loop than the
    float32 path does; an ignored ``acc_dtype`` would tie."""
    case = make_case(**spec)
    out32, _ = run(ref.reference, case)
    out64, lse64 = run(ref.reference, case, acc_dtype=np.float64)
    want, want_lse = run(ref.brute_force_fp64, case)
    err64 = np.abs(out64 - want).max()
    assert err64 <= 1.5e-7 and err64 <= 0.6 * np.abs(out32 - want).max()
    np.testing.assert_allclose(lse64, want_lse, atol=5e-7, rtol=0)


def test_f16_dequant_is_exact_for_power_of_two_scales():
    """Every e4m3fn value times 2^-k (k small) is an fp16 value, so the
    fp16-rounded path must equal the fp32 path bit for bit."""
    case = _power_of_two_case()
    out32, lse32 = run(ref.reference, case)
    out16, lse16 = run(ref.reference, case, round_kv_to=np.float16)
    assert np.array_equal(out16, out32) and np.array_equal(lse16, lse32)


def _torch_literal_reference(case):
    """The reference oracle's steps in torch (fp8 -> float -> * scale -> fp16,
    gather, GQA repeat, softmax, weighted V), causal over the newest q_len."""
    q_len = case["q_len"]
    query = torch.from_numpy(case["query"])
    kc = torch.from_numpy(case["key_cache"]).view(torch.float8_e4m3fn)
    vc = torch.from_numpy(case["value_cache"]).view(torch.float8_e4m3fn)
    hq, d = query.shape[1], query.shape[2]
    hkv = kc.shape[2]
    outs = []
    for b, length in enumerate(case["seq_lens"].tolist()):
        t = torch.arange(length)
        pages = torch.from_numpy(case["block_table"][b]).long()[t // 16]
        k = (kc[pages, t % 16].float() * float(case["k_scale"])).to(torch.float16).float()
        v = (vc[pages, t % 16].float() * float(case["v_scale"])).to(torch.float16).float()
        k = k.repeat_interleave(hq // hkv, dim=1)
        v = v.repeat_interleave(hq // hkv, dim=1)
        for i in range(q_len):
            lim = length - q_len + i + 1
            s = torch.einsum("hd,thd->ht", query[b * q_len + i], k[:lim]) * d ** -0.5
            outs.append(torch.einsum("ht,thd->hd", torch.softmax(s, dim=-1), v[:lim]))
    return torch.stack(outs).numpy()


def test_f16_dequant_matches_torch_literal_restatement():
    """Non-power-of-two scales: the fp16 rounding changes the result, and the
    oracle's rounded path matches torch's own fp16 cast of the same products.
    A rounding applied before the scale (exact, so a no-op) or to bf16 fails."""
    case = make_case(seed=22, batch=2, hq=6, hkv=2, d=128, lens=[50, 93], q_len=2)
    out32, _ = run(ref.reference, case)
    out16, _ = run(ref.reference, case, round_kv_to=np.float16)
    want = _torch_literal_reference(case)
    assert np.abs(out16 - out32).max() > 1e-6
    np.testing.assert_allclose(out16, want, atol=2e-6, rtol=0)
    assert np.abs(out32 - want).max() > 4 * np.abs(out16 - want).max()


def _reduced(name):
    """The configuration's head layout, scales and q_len on a few sequences."""
    import dataclasses

    import l20_pd_workloads as wl

    kw = {"c2_qwen2.5_coder_3b": dict(batch=4), "c3_qwen2.5_7b": dict(batch=16),
          "c4_llama3_8b_long": dict(batch=1, context=16384), "c5_llama3_70b_verify": dict(batch=3)}
    return dataclasses.replace(wl.CONFIGS[name], **kw.get(name, {}))


@pytest.mark.parametrize("name", ["c1_qwen2.5_0.5b", "c2_qwen2.5_coder_3b", "c3_qwen2.5_7b",
                                  "c4_llama3_8b_long", "c5_llama3_70b_verify"])
def test_reference_literal_f16_dequant_within_tolerance_of_fp32_oracle(name):
    """The reference's literal oracle and this fp32 oracle agree within the
    north-star tolerances (max-abs 1e-2, cosine 0.9999, LSE 1e-4 relative) on
    every configuration shape, so parity against either is the same claim."""
    import l20_pd_workloads as wl

    cfg = _reduced(name)
    inp = wl.make_inputs(cfg)

    def sc(x):
        return x if isinstance(x, float) else x.numpy()

    args = (inp["query"].float().numpy(), inp["key_cache"].view(torch.uint8).numpy(),
            inp["value_cache"].view(torch.uint8).numpy(), inp["block_table"].numpy(), inp["seq_lens"].numpy(),
            sc(inp["k_scale"]), sc(inp["v_scale"]))
    o32, l32 = ref.reference(*args, softmax_scale=inp["softmax_scale"], q_len=cfg.q_len)
    o16, l16 = ref.reference(*args, softmax_scale=inp["softmax_scale"], q_len=cfg.q_len, round_kv_to=np.float16)
    a = o32.reshape(-1, o32.shape[-1]).astype(np.float64)
    b = o16.reshape(-1, o16.shape[-1]).astype(np.float64)
    cos = (a * b).sum(-1) / np.maximum(np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1), 1e-30)
    assert np.abs(o32 - o16).max() <= 1e-2 / 10
    assert cos.min() >= 0.9999
    assert (np.abs(l32 - l16) / np.maximum(1.0, np.abs(l32))).max() <= 1e-4
