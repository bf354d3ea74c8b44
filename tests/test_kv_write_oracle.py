"""Pins of the KV-cache producer oracle (oracle/kv_write_ref.py) on the CPU."""

import numpy as np
import pytest
import torch

from oracle import kv_write_ref as kw
from oracle import paged_fp8_decode_ref as pd


def test_round_bf16_matches_torch_including_ties():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(20000).astype(np.float32) * np.float32(3.0)
    # exact ties between adjacent bf16 values and values just around them
    base = torch.randn(2000).to(torch.bfloat16).float().numpy()
    ulp = np.abs(base) * np.float32(2.0 ** -8)
    ties = np.concatenate([base + ulp / 2, base - ulp / 2, base + ulp / 2 * np.float32(1.0001)]).astype(np.float32)
    for v in (x, ties, np.array([0.0, -0.0, 1e-40, 3.0e38, -65504.0], np.float32)):
        want = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
        np.testing.assert_array_equal(kw.round_bf16(v).view(np.uint32), want.view(np.uint32))


def _complex_rope(x, theta, is_neox, rot):
    """float64 reference: each pair as a complex number times e^{i theta}."""
    x = np.asarray(x, dtype=np.float64)
    out = x.copy()
    half = rot // 2
    if is_neox:
        z = x[..., :half] + 1j * x[..., half:rot]
    else:
        z = x[..., 0:rot:2] + 1j * x[..., 1:rot:2]
    z = z * np.exp(1j * theta)[..., None, :]
    if is_neox:
        out[..., :half], out[..., half:rot] = z.real, z.imag
    else:
        out[..., 0:rot:2], out[..., 1:rot:2] = z.real, z.imag
    return out


@pytest.mark.parametrize("dtype,torch_dtype", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_round_to_matches_torch_casts(dtype, torch_dtype):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4000) * 100, rng.standard_normal(4000) * 1e-6,
                        [0.0, -0.0, 65504.0, 1e-8]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch_dtype).float().numpy()
    assert np.array_equal(kw.round_to(x, dtype), want)
    with pytest.raises(ValueError):
        kw.round_to(x, "fp8")


@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("rot,d", [(128, 128), (64, 128), (32, 64)])
def test_rope_matches_complex_rotation(is_neox, rot, d):
    rng = np.random.default_rng(rot + d + int(is_neox))
    x = rng.standard_normal((5, 3, d)).astype(np.float32)
    theta = rng.uniform(-np.pi, np.pi, (5, rot // 2))
    cs = np.concatenate([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32)
    got = kw.rope(x, cs, rot, is_neox)
    want = _complex_rope(x, theta.astype(np.float32).astype(np.float64), is_neox, rot)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(got[..., rot:], x[..., rot:])  # tail dims untouched


@pytest.mark.parametrize("is_neox", [True, False])
def test_rope_identity_and_composition(is_neox):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 2, 64)).astype(np.float32)
    ident = np.concatenate([np.ones((4, 32)), np.zeros((4, 32))], -1).astype(np.float32)
    np.testing.assert_array_equal(kw.rope(x, ident, 64, is_neox), x)
    theta = rng.uniform(-1, 1, (4, 32))
    one = np.concatenate([np.cos(theta), np.sin(theta)], -1).astype(np.float32)
    two = np.concatenate([np.cos(2 * theta), np.sin(2 * theta)], -1).astype(np.float32)
    np.testing.assert_allclose(kw.rope(kw.rope(x, one, 64, is_neox), one, 64, is_neox),
                               kw.rope(x, two, 64, is_neox), atol=2e-5)


def test_planted_pair_swap_is_caught():
    """A rotation with the pair layouts swapped (neox <-> interleaved) must disagree."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 2, 64)).astype(np.float32)
    theta = rng.uniform(-np.pi, np.pi, (3, 32))
    cs = np.concatenate([np.cos(theta), np.sin(theta)], -1).astype(np.float32)
    want = _complex_rope(x, theta.astype(np.float32).astype(np.float64), True, 64)
    assert not np.allclose(kw.rope(x, cs, 64, False), want, atol=1e-3)


def test_quantize_rows_per_tensor_and_per_head_match_the_pinned_quantiser():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((10, 4, 64)) * 3).astype(np.float32)
    s = kw.fp8_scales(x, per_head=False)
    codes, scale = pd.quantize_fp8_e4m3(x)
    assert np.float32(scale) == s[0]
    np.testing.assert_array_equal(kw.quantize_rows(x, s[0]), codes)
    sh = kw.fp8_scales(x, per_head=True)
    codes_h, scales_h = pd.quantize_fp8_e4m3_per_head(x, head_axis=1)
    np.testing.assert_array_equal(sh, scales_h)
    np.testing.assert_array_equal(kw.quantize_rows(x, sh), codes_h)


@pytest.mark.parametrize("cache_fp8", [True, False])
def test_rope_and_cache_scatter_round_trip(cache_fp8):
    rng = np.random.default_rng(3)
    T, Hq, Hkv, D, pages = 20, 8, 2, 64, 6
    q = kw.round_bf16(rng.standard_normal((T, Hq, D)).astype(np.float32))
    k = kw.round_bf16(rng.standard_normal((T, Hkv, D)).astype(np.float32))
    v = kw.round_bf16(rng.standard_normal((T, Hkv, D)).astype(np.float32))
    pos = rng.integers(0, 100, T)
    theta = rng.uniform(-3, 3, (100, D // 2))
    csc = kw.round_bf16(np.concatenate([np.cos(theta), np.sin(theta)], -1).astype(np.float32))
    slots = rng.permutation(pages * 16)[:T]
    slots[[3, 11]] = -1  # padding tokens are skipped
    if cache_fp8:
        kc = np.zeros((pages, 16, Hkv, D), np.uint8)
        vc = np.zeros_like(kc)
    else:
        kc = np.zeros((pages, 16, Hkv, D), np.float32)
        vc = np.zeros_like(kc)
    qo, ko, kc2, vc2 = kw.rope_and_cache(q, k, v, pos, csc, True, kc, vc, slots, dtype="bf16",
                                         cache_fp8=cache_fp8, k_scale=0.01, v_scale=0.02)
    np.testing.assert_array_equal(qo, kw.round_bf16(kw.rope(q, csc[pos], D, True)))
    for t, s in enumerate(slots):
        if s < 0:
            continue
        got_k, got_v = kc2[s // 16, s % 16], vc2[s // 16, s % 16]
        if cache_fp8:
            np.testing.assert_array_equal(got_k, kw.quantize_rows(ko[t], 0.01))
            np.testing.assert_array_equal(got_v, kw.quantize_rows(v[t], 0.02))
        else:
            np.testing.assert_array_equal(got_k, ko[t])
            np.testing.assert_array_equal(got_v, v[t])
    written = np.zeros(pages * 16, bool)
    written[slots[slots >= 0]] = True
    untouched = ~written.reshape(pages, 16)
    assert np.all(kc2[untouched] == 0) and np.all(vc2[untouched] == 0)
