"""Pins the oracle's SiLU(gate) * up (cuda/silu_kernel.cu:6-18).

Pinned by scipy's expit (an independent sigmoid) in float64, the identity
silu(x) - silu(-x) = x, silu(0) = 0, up = 1 giving silu itself, and the
saturation limits (very negative gate -> -0.0, large gate -> gate * up).
"""
import numpy as np
from scipy.special import expit

import oracle
import testutil as tu


def test_vs_expit_fp32():
    r = tu.rng(51)
    g = tu.normal(r, (100000,), 0.0, 2.0, np.float32)
    u = tu.normal(r, (100000,), 0.0, 2.0, np.float32)
    expect = g.astype(np.float64) * expit(g.astype(np.float64)) * u.astype(np.float64)
    tu.assert_f32_close(oracle.swiglu(g, u), expect, rel=1e-6, floor=1e-30)


def test_vs_expit_fp16():
    r = tu.rng(52)
    g = tu.normal(r, (200000,), 0.0, 2.0)
    u = tu.normal(r, (200000,), 0.0, 2.0)
    expect = (g.astype(np.float64) * expit(g.astype(np.float64)) * u.astype(np.float64))
    tu.assert_f16_close(oracle.swiglu(g, u), expect.astype(np.float16), max_ulp=1)


def test_odd_identity_and_zero():
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    one = np.ones_like(x)
    s_pos = oracle.swiglu(x, one).astype(np.float64)
    s_neg = oracle.swiglu(-x, one).astype(np.float64)
    assert np.max(np.abs((s_pos - s_neg) - x)) < 1e-5
    assert oracle.swiglu(np.zeros(4, np.float32), np.ones(4, np.float32)).tolist() == [0.0] * 4


def test_saturation_limits():
    g = np.array([-65504.0, -1000.0, -200.0, 100.0, 65504.0], np.float32)
    u = np.array([3.0, 1.0, 2.0, 0.5, 1.0], np.float32)
    out = oracle.swiglu(g, u)
    assert np.all(out[:3] == 0) and np.all(np.signbit(out[:3]))  # -0.0
    assert out[3] == 50.0 and out[4] == 65504.0
    g16 = np.array([-65504.0, -20.0, 65504.0], np.float16)
    out16 = oracle.swiglu(g16, np.ones(3, np.float16))
    assert out16[0] == 0 and np.signbit(out16[0])
    assert out16[2] == np.float16(65504.0)
