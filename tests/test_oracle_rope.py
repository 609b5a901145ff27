"""Pins the oracle's interleaved RoPE (cuda/rope_kernel.cu:8-50).

Pinned by: theta_i against numpy's float64 power (theta_0 == 1 exactly), the
rotation restated as complex multiplication with numpy's complex exp on the
reference's fp32 angle (exposes a sign or direction error), one-hot inputs that
fix the interleaved (2i, 2i+1) pairing (not the half-split NeoX layout),
pos = 0 identity, norm preservation, and the K heads sharing the Q schedule.
"""
import numpy as np

import oracle
import testutil as tu

HD = 128
BASE = 500000.0


def f32_angles(pos, head_dim=HD, base=BASE):
    th = np.array([oracle.rope_theta(base, i, head_dim) for i in range(head_dim // 2)],
                  np.float32)
    return np.float32(pos) * th  # fp32 product, as the reference forms it


def test_theta_table():
    th = np.array([oracle.rope_theta(BASE, i, HD) for i in range(HD // 2)], np.float32)
    assert th[0] == 1.0
    exact = BASE ** (-2.0 * np.arange(HD // 2) / HD)
    # correctly rounded: within half an fp32 ulp of the float64 value
    ulp = np.spacing(th.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(th.astype(np.float64) - exact) <= 0.5 * ulp * (1 + 1e-9))


def test_complex_statement():
    r = tu.rng(41)
    T, nh, nkv = 24, 4, 2
    q = tu.normal(r, (T, nh * HD), dtype=np.float32)
    k = tu.normal(r, (T, nkv * HD), dtype=np.float32)
    pos = r.integers(0, 8192, size=T).astype(np.int32)
    q2, k2 = oracle.rope_rows(q, k, HD, pos, 0, BASE)
    for src, dst, nhd in ((q, q2, nh), (k, k2, nkv)):
        z = src.reshape(T, nhd, HD // 2, 2).astype(np.float64)
        zc = z[..., 0] + 1j * z[..., 1]
        a = np.stack([f32_angles(p) for p in pos]).astype(np.float64)[:, None, :]
        rot = zc * np.exp(1j * a)
        got = dst.reshape(T, nhd, HD // 2, 2).astype(np.float64)
        err = np.abs(got[..., 0] + 1j * got[..., 1] - rot)
        assert np.max(err / np.maximum(np.abs(zc), 1e-30)) < 1e-6


def test_interleaved_pairing_one_hot():
    i, h = 5, 1
    q = np.zeros((1, 2 * HD), np.float32)
    q[0, h * HD + 2 * i] = 1.0
    k = np.zeros((1, HD), np.float32)
    q2, _ = oracle.rope_rows(q, k, HD, np.array([1000], np.int32), 0, BASE)
    a = float(f32_angles(1000)[i])
    nz = np.nonzero(q2[0])[0]
    assert set(nz) <= {h * HD + 2 * i, h * HD + 2 * i + 1}
    assert abs(q2[0, h * HD + 2 * i] - np.cos(a)) < 1e-7
    assert abs(q2[0, h * HD + 2 * i + 1] - np.sin(a)) < 1e-7


def test_pos0_identity_bit_exact():
    r = tu.rng(42)
    for dt in (np.float32, np.float16):
        q = tu.normal(r, (3, 4 * HD), dtype=dt)
        k = tu.normal(r, (3, 2 * HD), dtype=dt)
        q2, k2 = oracle.rope_rows(q, k, HD, np.zeros(3, np.int32), 0, BASE)
        assert tu.bits_equal(q2, q) and tu.bits_equal(k2, k)


def test_norm_preserved_and_kv_schedule():
    r = tu.rng(43)
    x = tu.normal(r, (8, HD), dtype=np.float32)
    q = np.tile(x, (1, 3))
    k = x.copy()
    pos = r.integers(0, 8192, size=8).astype(np.int32)
    q2, k2 = oracle.rope_rows(q, k, HD, pos, 0, BASE)
    for h in range(3):
        assert tu.bits_equal(q2[:, h * HD:(h + 1) * HD], k2)
    n0 = np.hypot(x[:, 0::2], x[:, 1::2]).astype(np.float64)
    n1 = np.hypot(k2[:, 0::2], k2[:, 1::2]).astype(np.float64)
    assert np.max(np.abs(n1 - n0) / np.maximum(n0, 1e-30)) < 1e-6


def test_positions_default_to_pos0_plus_t():
    r = tu.rng(44)
    q = tu.normal(r, (5, HD), dtype=np.float32)
    k = tu.normal(r, (5, HD), dtype=np.float32)
    a = oracle.rope_rows(q, k, HD, None, 37, BASE)
    b = oracle.rope_rows(q, k, HD, np.arange(37, 42, dtype=np.int32), 0, BASE)
    assert tu.bits_equal(a[0], b[0]) and tu.bits_equal(a[1], b[1])


def test_fp16_vs_fp32_path():
    r = tu.rng(45)
    q = tu.normal(r, (16, 2 * HD))
    k = tu.normal(r, (16, HD))
    pos = r.integers(0, 8192, size=16).astype(np.int32)
    q16, k16 = oracle.rope_rows(q, k, HD, pos, 0, BASE)
    q32, k32 = oracle.rope_rows(q.astype(np.float32), k.astype(np.float32), HD, pos, 0, BASE)
    assert tu.bits_equal(q16, q32.astype(np.float16)) and tu.bits_equal(k16, k32.astype(np.float16))
