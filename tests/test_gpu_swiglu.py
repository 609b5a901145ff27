"""GPU parity: SwiGLU (fp16 rows and the fp32 drop-in) and residual add.

Bar: fp16 within 2 ulp of the oracle (the fp16 kernel uses the hardware exp2 /
reciprocal; its fp32 value is within ~2e-6 relative of the exact expression,
so it lands on the oracle's fp16 value or one ulp away), fp32 within 1e-5
relative, residual add bit-exact.
"""
import os

import numpy as np
import pytest
import torch

import jinf_amd
import oracle
import testutil as tu
from gpu_util import dev as to_dev
from gpu_util import host, say

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_config3b_full(dev):
    say("config 3b: SwiGLU fp16 [2048, 14336], gate/up ~ N(0, 2)")
    r = tu.rng(33)
    g = tu.normal(r, (2048, 14336), 0.0, 2.0)
    u = tu.normal(r, (2048, 14336), 0.0, 2.0)
    oracle.set_threads(8)
    ref = oracle.swiglu(g, u)
    oracle.set_threads(1)
    got = host(jinf_amd.swiglu(to_dev(g), to_dev(u)))
    w = tu.assert_f16_close(got, ref, 2, "swiglu")
    say(f"worst ulp {w}, bit-identical fraction {np.mean(got.view(np.uint16) == ref.view(np.uint16)):.6f}")


def test_fixture(dev):
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    got = host(jinf_amd.swiglu(to_dev(g["sw_gate"]), to_dev(g["sw_up"])))
    tu.assert_f16_close(got, g["sw_out"], 2, "fixture")


def test_edge_values_fp16(dev):
    say("edge gates: +-65504, +-inf, NaN, -20, 0, subnormal")
    g = np.array([-65504, -20, -0.0, 0.0, 6e-8, 65504, np.inf, -np.inf, np.nan, -16.0, 12.0, -88.0,
                  1.0, -1.0, 3.0, -3.0], np.float16)
    u = np.array([3, 1, 1, 1, 1, 1, 2, 2, 1, 1000, -1, 7, 1, 1, -2, 65504], np.float16)
    ref = oracle.swiglu(g, u)
    got = host(jinf_amd.swiglu(to_dev(g), to_dev(u)))
    tu.assert_f16_close(got, ref, 2, "edges")
    assert np.signbit(got[0]) and got[0] == 0  # -0.0 survives


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 14336, 28672 * 64 + 3])
def test_drop_in_fp32_in_place(dev, n):
    say(f"drop-in jinf_cuda_silu_mul n={n}, output == gate")
    r = tu.rng(n)
    g = tu.normal(r, (n,), 0.0, 2.0, np.float32)
    u = tu.normal(r, (n,), 0.0, 2.0, np.float32)
    ref = oracle.swiglu(g, u)
    gd = to_dev(g)
    jinf_amd.cuda_silu_mul(gd, gd, to_dev(u))
    tu.assert_f32_close(host(gd), ref, 1e-5, 1e-30, f"n={n}")


def test_strided_gate_up_halves(dev):
    say("gate/up as the two halves of a fused [T, 2*ff] buffer, out == up")
    r = tu.rng(35)
    T, ff = 64, 28672
    gu = tu.normal(r, (T, 2 * ff), 0.0, 2.0)
    ref = oracle.swiglu(np.ascontiguousarray(gu[:, :ff]), np.ascontiguousarray(gu[:, ff:]))
    d = to_dev(gu)
    jinf_amd.swiglu(d[:, :ff], d[:, ff:], out=d[:, ff:])
    got = host(d)
    tu.assert_f16_close(np.ascontiguousarray(got[:, ff:]), ref, 2, "strided")
    assert tu.bits_equal(got[:, :ff], gu[:, :ff])


@pytest.mark.parametrize("dt", [np.float16, np.float32])
@pytest.mark.parametrize("shape", [(64, 8192), (3, 1001), (1, 5)])
def test_residual_add_bit_exact(dev, dt, shape):
    say(f"residual add {np.dtype(dt).name} {shape}")
    r = tu.rng(shape[1])
    a = tu.normal(r, shape, dtype=dt)
    b = tu.normal(r, shape, dtype=dt)
    b.reshape(-1)[::97] = np.array(6e-8 if dt == np.float16 else 1e-40, dtype=dt)  # subnormals
    ref = oracle.residual_add(a, b)
    ad = to_dev(a)
    jinf_amd.residual_add(ad, to_dev(b))
    assert tu.bits_equal(host(ad), ref)
    if dt == np.float32:
        ad = to_dev(a[0])
        jinf_amd.cuda_residual_add(ad, to_dev(b[0]))
        assert tu.bits_equal(host(ad), ref[0])
