"""Pins the oracle's GQA decode attention (cuda/attention_kernel.cu:25-96).

Pinned by: scipy's softmax over numpy float64 matrix products (independent
library routines); closed forms -- one cached position returns its value row
exactly, identical keys give the mean of the values, one dominant key returns
its value row; the GQA head mapping (query head h reads kv head
h / (n_heads / n_heads_kv)) through kv heads holding distinct constants; the
masked tail (NaN past each length) is never read; fp16 and fp32 caches holding
the same values agree.
"""
import numpy as np
from scipy.special import softmax

import oracle
import testutil as tu


def _np_attention(q, k, v, lens, nh, nkv, hd, scale):
    n_seq = q.shape[0]
    g = nh // nkv
    out = np.zeros((n_seq, nh * hd))
    for s in range(n_seq):
        L = lens[s]
        K = k[s, :L].astype(np.float64).reshape(L, nkv, hd)
        V = v[s, :L].astype(np.float64).reshape(L, nkv, hd)
        for h in range(nh):
            qh = q[s, h * hd:(h + 1) * hd].astype(np.float64)
            p = softmax(K[:, h // g, :] @ qh * scale)
            out[s, h * hd:(h + 1) * hd] = p @ V[:, h // g, :]
    return out


def _cache(r, n_seq, ctx, nkv, hd, dtype=np.float32):
    return (tu.normal(r, (n_seq, ctx, nkv * hd), 0.0, 1.0, np.float32).astype(dtype),
            tu.normal(r, (n_seq, ctx, nkv * hd), 0.0, 1.0, np.float32).astype(dtype))


def test_vs_scipy_softmax_restatement():
    r = tu.rng(101)
    n_seq, ctx, nh, nkv, hd = 3, 300, 8, 2, 64
    k, v = _cache(r, n_seq, ctx, nkv, hd)
    q = tu.normal(r, (n_seq, nh * hd), 0.0, 1.0, np.float32)
    lens = np.array([1, 300, 157], np.int32)
    out, a = oracle.attention(q, k, v, lens, nh, nkv, hd)
    ref = _np_attention(q, k, v, lens, nh, nkv, hd, 1.0 / np.sqrt(hd))
    assert np.all(np.abs(out - ref) <= 1e-7 * a + 1e-30)


def test_single_position_returns_value_row():
    r = tu.rng(102)
    k, v = _cache(r, 2, 16, 4, 128)
    q = tu.normal(r, (2, 8 * 128), 0.0, 3.0, np.float32)
    out, _ = oracle.attention(q, k, v, [1, 1], 8, 4, 128)
    for h in range(8):
        assert tu.bits_equal(out[:, h * 128:(h + 1) * 128], v[:, 0, (h // 2) * 128:(h // 2 + 1) * 128])


def test_identical_keys_give_the_mean_value():
    r = tu.rng(103)
    k, v = _cache(r, 1, 50, 1, 32)
    k[:] = k[:, :1]
    q = tu.normal(r, (1, 4 * 32), 0.0, 1.0, np.float32)
    out, _ = oracle.attention(q, k, v, [50], 4, 1, 32)
    mean = v[0].astype(np.float64).mean(axis=0)
    for h in range(4):
        assert np.allclose(out[0, h * 32:(h + 1) * 32], mean, rtol=1e-6, atol=1e-7)


def test_dominant_key_selects_its_value():
    r = tu.rng(104)
    k, v = _cache(r, 1, 40, 1, 16)
    q = np.ones((1, 16), np.float32)
    k[0, 17] = 100.0  # score 100 * 16 / 4 = 400 against O(1) for the rest
    out, _ = oracle.attention(q, k, v, [40], 1, 1, 16)
    assert np.allclose(out[0], v[0, 17], rtol=0, atol=1e-30)


def test_gqa_head_mapping():
    r = tu.rng(105)
    nh, nkv, hd = 12, 3, 8
    k, v = _cache(r, 1, 10, nkv, hd)
    for j in range(nkv):
        v[0, :, j * hd:(j + 1) * hd] = float(j + 1)
    q = tu.normal(r, (1, nh * hd), 0.0, 1.0, np.float32)
    out, _ = oracle.attention(q, k, v, [10], nh, nkv, hd)
    for h in range(nh):
        assert np.allclose(out[0, h * hd:(h + 1) * hd], h // (nh // nkv) + 1, rtol=1e-12)


def test_masked_tail_is_not_read_and_fp16_cache_matches():
    r = tu.rng(106)
    k, v = _cache(r, 2, 64, 2, 32, np.float16)
    lens = np.array([5, 33], np.int32)
    q = tu.normal(r, (2, 4 * 32), 0.0, 1.0, np.float32)
    k32, v32 = k.astype(np.float32), v.astype(np.float32)
    for s, L in enumerate(lens):
        k[s, L:] = np.nan
        v[s, L:] = np.nan
    out16, _ = oracle.attention(q, k, v, lens, 4, 2, 32)
    out32, _ = oracle.attention(q, k32, v32, lens, 4, 2, 32)
    assert np.all(np.isfinite(out16))
    assert tu.bits_equal(out16, out32)
