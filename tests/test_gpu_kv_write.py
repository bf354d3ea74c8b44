"""GPU parity of the paged KV-cache producer (RoPE + fp8/16-bit paged write)
against oracle/kv_write_ref.py: bit-exact (byte and integer work)."""

import ctypes

import numpy as np
import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    import l20_paged_decode  # noqa: F401


def _np(t):
    return t.float().cpu().numpy()


def _dtype_name(dt):
    return "bf16" if dt == torch.bfloat16 else "fp16"


def _kv_args(key, value, positions, cs, key_cache, value_cache, slots, *, rot, neox=True, query=None,
             k_scale=1.0, v_scale=1.0):
    import l20_pd_cabi as cabi

    a = cabi.L20PdKvWriteArgs()
    if query is not None:
        a.query, a.q_stride_token, a.q_stride_head, a.num_q_heads = (query.data_ptr(), query.stride(0),
                                                                     query.stride(1), query.shape[1])
    a.key, a.k_stride_token, a.k_stride_head = key.data_ptr(), key.stride(0), key.stride(1)
    a.value, a.v_stride_token, a.v_stride_head = value.data_ptr(), value.stride(0), value.stride(1)
    a.dtype = cabi.L20_PD_BF16 if key.dtype == torch.bfloat16 else cabi.L20_PD_FP16
    a.positions = positions.data_ptr()
    if cs is not None:
        a.cos_sin_cache, a.cs_stride_position = cs.data_ptr(), cs.stride(0)
        a.cs_dtype = {torch.bfloat16: cabi.L20_PD_BF16, torch.float16: cabi.L20_PD_FP16,
                      torch.float32: cabi.L20_PD_FP32}[cs.dtype]
    a.rotary_dim, a.is_neox = rot, int(neox)
    a.slot_mapping = slots.data_ptr()
    a.key_cache, a.value_cache = key_cache.data_ptr(), value_cache.data_ptr()
    a.kc_stride_page, a.kc_stride_token, a.kc_stride_head = key_cache.stride()[:3]
    a.vc_stride_page, a.vc_stride_token, a.vc_stride_head = value_cache.stride()[:3]
    a.num_pages = key_cache.shape[0]
    a.cache_dtype = (cabi.L20_PD_KV_FP8_E4M3 if key_cache.dtype == torch.float8_e4m3fn else
                     (cabi.L20_PD_KV_BF16 if key_cache.dtype == torch.bfloat16 else cabi.L20_PD_KV_FP16))
    a.k_scale, a.v_scale = k_scale, v_scale
    a.num_tokens, a.num_kv_heads, a.head_dim = key.shape
    return a


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("scale", [1.0, 0.37, 1.0 / 448, 3e-3])
def test_fp8_quantiser_on_every_finite_16bit_value(dtype, scale):
    """rotary_dim 0 through the C ABI: the cache bytes are RNE_e4m3fn(clamp(x / scale))
    for all 2^16 bit patterns of the model dtype (NaN/inf excluded)."""
    import l20_pd_cabi as cabi
    from oracle import kv_write_ref as kw

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    vals = bits.view(dtype)
    vals = vals[torch.isfinite(vals.float())]
    d = 64
    n = (vals.numel() // d) * d
    key = vals[:n].reshape(-1, 1, d).cuda()
    T = key.shape[0]
    value = key.flip(0).contiguous()
    pages = (T + 15) // 16
    kc = torch.zeros(pages, 16, 1, d, dtype=torch.float8_e4m3fn, device="cuda")
    vc = torch.zeros_like(kc)
    slots = torch.arange(T, dtype=torch.int64, device="cuda")
    pos = torch.zeros(T, dtype=torch.int64, device="cuda")
    a = _kv_args(key, value, pos, None, kc, vc, slots, rot=0, k_scale=scale, v_scale=scale)
    lib = cabi.load()
    assert lib.l20_pd_rope_and_cache(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0, \
        cabi.last_error(lib)
    torch.cuda.synchronize()
    want_k = kw.quantize_rows(_np(key), np.float32(scale))
    want_v = kw.quantize_rows(_np(value), np.float32(scale))
    got_k = kc.view(torch.uint8).cpu().numpy().reshape(-1, 1, d)[:T]
    got_v = vc.view(torch.uint8).cpu().numpy().reshape(-1, 1, d)[:T]
    np.testing.assert_array_equal(got_k, want_k)
    np.testing.assert_array_equal(got_v, want_v)


def _case(T, hq, hkv, d, rot, dtype, cs_dtype, seed, pages=None):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, hq, d, generator=g) * 2).to(dtype)
    k = (torch.randn(T, hkv, d, generator=g) * 2).to(dtype)
    v = (torch.randn(T, hkv, d, generator=g) * 2).to(dtype)
    max_pos = 4096
    theta = torch.rand(max_pos, rot // 2, generator=g, dtype=torch.float64) * 6.28 - 3.14
    cs = torch.cat([theta.cos(), theta.sin()], dim=-1).to(cs_dtype)
    pos = torch.randint(0, max_pos, (T,), generator=g)
    pages = pages or (T + 15) // 16 + 3
    slots = torch.randperm(pages * 16, generator=g)[:T]
    slots[torch.randperm(T, generator=g)[: max(1, T // 10)]] = -1  # padding tokens
    return dict(q=q, k=k, v=v, cs=cs, pos=pos, slots=slots, pages=pages)


ROPE = [
    # T, hq, hkv, d, rot, neox
    (37, 8, 2, 128, 128, True),
    (37, 8, 2, 128, 128, False),
    (20, 4, 4, 128, 64, True),
    (33, 16, 8, 64, 32, False),
    (5, 32, 8, 256, 256, True),
    (19, 6, 3, 96, 96, True),     # 12 lanes a row: 5 rows a wave, 4 idle lanes
    (21, 4, 2, 36, 24, False),    # head_dim % 8 != 0: the general path
    (15, 4, 2, 32, 24, True),     # neox halves not lane-aligned: the general path
]


@pytest.mark.parametrize("spec", ROPE, ids=[f"T{s[0]}_h{s[1]}x{s[2]}_d{s[3]}_r{s[4]}_{'neox' if s[5] else 'gptj'}"
                                           for s in ROPE])
@pytest.mark.parametrize("dtype,cs_dtype", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "fp16_cs32"])
@pytest.mark.parametrize("cache", ["fp8", "fp8_per_head", "model"])
def test_rope_and_cache_bit_exact(spec, dtype, cs_dtype, cache):
    from oracle import kv_write_ref as kw
    import l20_rope_kv

    T, hq, hkv, d, rot, neox = spec
    c = _case(T, hq, hkv, d, rot, dtype, cs_dtype, seed=T * 7 + d)
    fp8 = cache != "model"
    cache_dtype = torch.float8_e4m3fn if fp8 else dtype
    kc = torch.zeros(c["pages"], 16, hkv, d, dtype=cache_dtype).cuda()
    vc = torch.zeros_like(kc)
    q, k, v = c["q"].cuda(), c["k"].cuda(), c["v"].cuda()
    ks = vs = 1.0
    ksph = vsph = None
    if cache == "fp8":
        ks, vs = 0.031, 0.017
    elif cache == "fp8_per_head":
        ksph = torch.linspace(0.01, 0.05, hkv, dtype=torch.float32).cuda()
        vsph = torch.linspace(0.02, 0.03, hkv, dtype=torch.float32).cuda()
    q_in, k_in = _np(q), _np(k)
    l20_rope_kv.l20_rope_and_cache(q, k, v, c["pos"].cuda(), c["cs"].cuda(), neox, kc, vc, c["slots"].cuda(),
                                   k_scale=ks, v_scale=vs, k_scale_per_head=ksph, v_scale_per_head=vsph)
    torch.cuda.synchronize()
    kc0 = np.zeros(kc.shape, np.uint8 if fp8 else np.float32)
    want_q, want_k, want_kc, want_vc = kw.rope_and_cache(
        q_in, k_in, _np(v), c["pos"].numpy(), _np(c["cs"]), neox, kc0, kc0.copy(), c["slots"].numpy(),
        dtype=_dtype_name(dtype), cache_fp8=fp8,
        k_scale=ksph.cpu().numpy() if ksph is not None else ks,
        v_scale=vsph.cpu().numpy() if vsph is not None else vs)
    np.testing.assert_array_equal(_np(q), want_q)
    np.testing.assert_array_equal(_np(k), want_k)
    if fp8:
        np.testing.assert_array_equal(kc.view(torch.uint8).cpu().numpy(), want_kc)
        np.testing.assert_array_equal(vc.view(torch.uint8).cpu().numpy(), want_vc)
    else:
        np.testing.assert_array_equal(_np(kc), want_kc)
        np.testing.assert_array_equal(_np(vc), want_vc)


@pytest.mark.parametrize("page", [32, 48])
def test_rope_and_cache_pages_of_a_multiple_of_16_tokens(page):
    """Caches of page-token blocks (vLLM's block size passes through): slot s is
    row s % page of block s // page, bit-exact against the oracle."""
    from oracle import kv_write_ref as kw
    import l20_rope_kv

    T, hq, hkv, d, rot = 37, 8, 2, 128, 128
    c = _case(T, hq, hkv, d, rot, torch.bfloat16, torch.bfloat16, seed=page)
    pages = (c["pages"] * 16 + page - 1) // page
    kc = torch.zeros(pages, page, hkv, d, dtype=torch.float8_e4m3fn).cuda()
    vc = torch.zeros_like(kc)
    q, k, v = c["q"].cuda(), c["k"].cuda(), c["v"].cuda()
    q_in, k_in = _np(q), _np(k)
    l20_rope_kv.l20_rope_and_cache(q, k, v, c["pos"].cuda(), c["cs"].cuda(), True, kc, vc, c["slots"].cuda(),
                                   k_scale=0.031, v_scale=0.017)
    torch.cuda.synchronize()
    kc0 = np.zeros(kc.shape, np.uint8)
    want_q, want_k, want_kc, want_vc = kw.rope_and_cache(
        q_in, k_in, _np(v), c["pos"].numpy(), _np(c["cs"]), True, kc0, kc0.copy(), c["slots"].numpy(),
        dtype="bf16", cache_fp8=True, k_scale=0.031, v_scale=0.017)
    np.testing.assert_array_equal(_np(q), want_q)
    np.testing.assert_array_equal(kc.view(torch.uint8).cpu().numpy(), want_kc)
    np.testing.assert_array_equal(vc.view(torch.uint8).cpu().numpy(), want_vc)
    # padded blocks (block stride != page token strides) are refused
    padded = torch.zeros(pages, page + 16, hkv, d, dtype=torch.float8_e4m3fn).cuda()[:, :page]
    with pytest.raises(RuntimeError, match="contiguously"):
        l20_rope_kv.l20_rope_and_cache(None, k, v, c["pos"].cuda(), c["cs"].cuda(), True, padded, padded,
                                       c["slots"].cuda(), k_scale=0.031, v_scale=0.017)


def test_rope_and_cache_rows_only_8_byte_aligned():
    """Q/K/V rows 8-byte but not 16-byte aligned (views at an offset of four
    elements) take the general path and give the same bytes."""
    from oracle import kv_write_ref as kw
    import l20_rope_kv

    T, hq, hkv, d = 23, 8, 2, 64
    c = _case(T, hq, hkv, d, 64, torch.bfloat16, torch.bfloat16, seed=5)
    def offset_view(x):
        big = torch.zeros(x.shape[0], x.shape[1], d + 4, dtype=x.dtype)
        big[..., 4:] = x
        return big.cuda()[..., 4:]
    q, k, v = offset_view(c["q"]), offset_view(c["k"]), offset_view(c["v"])
    assert q.data_ptr() % 16 == 8
    kc = torch.zeros(c["pages"], 16, hkv, d, dtype=torch.float8_e4m3fn).cuda()
    vc = torch.zeros_like(kc)
    q_in, k_in, v_in = _np(q), _np(k), _np(v)
    l20_rope_kv.l20_rope_and_cache(q, k, v, c["pos"].cuda(), c["cs"].cuda(), True, kc, vc, c["slots"].cuda(),
                                   k_scale=0.03, v_scale=0.02)
    torch.cuda.synchronize()
    kc0 = np.zeros(kc.shape, np.uint8)
    want_q, want_k, want_kc, want_vc = kw.rope_and_cache(
        q_in, k_in, v_in, c["pos"].numpy(), _np(c["cs"]), True, kc0, kc0.copy(), c["slots"].numpy(),
        dtype="bf16", cache_fp8=True, k_scale=0.03, v_scale=0.02)
    np.testing.assert_array_equal(_np(q), want_q)
    np.testing.assert_array_equal(_np(k), want_k)
    np.testing.assert_array_equal(kc.view(torch.uint8).cpu().numpy(), want_kc)
    np.testing.assert_array_equal(vc.view(torch.uint8).cpu().numpy(), want_vc)


@pytest.mark.parametrize("per_head", [True, False])
def test_fp8_scales_match_oracle(per_head):
    from oracle import kv_write_ref as kw
    import l20_rope_kv

    c = _case(300, 8, 4, 128, 128, torch.bfloat16, torch.bfloat16, seed=3)
    kc = torch.zeros(c["pages"], 16, 4, 128, dtype=torch.float8_e4m3fn).cuda()
    k = c["k"].cuda()
    ks, vs = l20_rope_kv.l20_kv_fp8_scales(k, c["v"].cuda(), c["pos"].cuda(), c["cs"].cuda(), True, kc, kc.clone(),
                                           c["slots"].cuda(), per_head=per_head)
    torch.cuda.synchronize()
    stored = c["slots"].numpy() >= 0
    k_rot = kw.round_bf16(kw.rope(_np(c["k"]), _np(c["cs"])[c["pos"].numpy()], 128, True))[stored]
    want_k = kw.fp8_scales(k_rot, per_head)
    want_v = kw.fp8_scales(_np(c["v"])[stored], per_head)
    if not per_head:
        want_k, want_v = np.repeat(want_k, 4), np.repeat(want_v, 4)
    np.testing.assert_array_equal(ks.cpu().numpy(), want_k)
    np.testing.assert_array_equal(vs.cpu().numpy(), want_v)
    np.testing.assert_array_equal(_np(k), _np(c["k"]))  # the scale pass leaves K untouched


def test_produced_fp8_cache_feeds_the_decode_op():
    """Producer -> consumer: decode tokens written by rope_and_cache (per-head scales from
    kv_fp8_scales) and compare the attention with the oracle over the same bytes."""
    import l20_rope_kv

    B, hq, hkv, d, L = 3, 16, 2, 128, 100
    T = B * L
    g = torch.Generator().manual_seed(21)
    k = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).cuda()
    theta = torch.rand(L, d // 2, generator=g, dtype=torch.float64) * 3
    cs = torch.cat([theta.cos(), theta.sin()], -1).to(torch.float32).cuda()
    pos = torch.arange(L).repeat(B).cuda()
    pages_per = (L + 15) // 16
    perm = torch.randperm(B * pages_per + 4, generator=g).to(torch.int32)
    table = perm[: B * pages_per].reshape(B, pages_per).cuda()
    slots = (table.long()[torch.arange(B).repeat_interleave(L).cuda(), pos // 16] * 16 + pos % 16).contiguous()
    kc = torch.zeros(B * pages_per + 4, 16, hkv, d, dtype=torch.float8_e4m3fn, device="cuda")
    vc = torch.zeros_like(kc)
    ks, vs = l20_rope_kv.l20_kv_fp8_scales(k, v, pos, cs, True, kc, vc, slots)
    l20_rope_kv.l20_rope_and_cache(None, k, v, pos, cs, True, kc, vc, slots, k_scale_per_head=ks, v_scale_per_head=vs)
    torch.cuda.synchronize()
    inp = {
        "query": torch.randn(B, hq, d, generator=g).to(torch.bfloat16).cuda(), "key_cache": kc, "value_cache": vc,
        "block_table": table, "seq_lens": torch.full((B,), L, dtype=torch.int32, device="cuda"),
        "k_scale": ks, "v_scale": vs, "softmax_scale": d ** -0.5, "q_len": 1, "max_seq_len": L,
    }
    H.compare(*H.run_op(inp, 64), *H.run_oracle(inp))
