"""Pins the oracle's RMSNorm and fused residual + RMSNorm
(cuda/rmsnorm_kernel.cu:9-61, cuda/matmul_kernels.cu:189-194,
src/engine.cpp:466->487).

Pinned by closed forms (constant, zero and one-hot rows: these expose a missing
eps, n-1 instead of n, a missing weight), a float64 numpy statement of
y = x / sqrt(mean(x^2) + eps) * w, scale invariance, the identity
fused == residual add then norm, and the distance of the reference's own fp32
summation order from the fp64 sum the oracle uses.
"""
import os

import numpy as np

import oracle
import testutil as tu

HERE = os.path.dirname(os.path.abspath(__file__))
EPS = 1e-5


def np_rms(x, w, eps=EPS):
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w.astype(np.float64)


def test_constant_rows_closed_form():
    n = 4096
    w = tu.normal(tu.rng(31), (n,), 1.0, 0.05, np.float32)
    for c in (1e-3, 0.5, -3.0, 100.0):
        x = np.full((1, n), c, np.float32)
        y = oracle.rmsnorm_rows(x, w, EPS)
        expect = c / np.sqrt(np.float64(c) ** 2 + EPS) * w.astype(np.float64)
        tu.assert_f32_close(y[0], expect, rel=1e-6, what=f"c={c}")


def test_zero_row_is_zero():
    y = oracle.rmsnorm_rows(np.zeros((2, 512), np.float32), np.ones(512, np.float32), EPS)
    assert np.all(y == 0)


def test_one_hot():
    n, k, a = 1000, 123, 7.0
    x = np.zeros((1, n), np.float32)
    x[0, k] = a
    w = tu.normal(tu.rng(32), (n,), 1.0, 0.05, np.float32)
    y = oracle.rmsnorm_rows(x, w, EPS)
    assert np.all(np.delete(y[0], k) == 0)
    tu.assert_f32_close(y[0, k], a / np.sqrt(a * a / n + EPS) * np.float64(w[k]), rel=1e-6)


def test_random_vs_float64_statement():
    r = tu.rng(33)
    for n in (4096, 8192, 1000, 77):
        x = tu.normal(r, (16, n), 0.0, 1.0, np.float32)
        w = tu.normal(r, (n,), 1.0, 0.05, np.float32)
        tu.assert_f32_close(oracle.rmsnorm_rows(x, w, EPS), np_rms(x, w), rel=1e-6, floor=1e-6)
        w16 = w.astype(np.float16)
        tu.assert_f32_close(oracle.rmsnorm_rows(x, w16, EPS), np_rms(x, w16), rel=1e-6, floor=1e-6)


def test_fp16_vs_float64_statement():
    r = tu.rng(34)
    x = tu.normal(r, (64, 4096))
    w = tu.normal(r, (4096,), 1.0, 0.05)
    y = oracle.rmsnorm_rows(x, w, EPS)
    tu.assert_f16_close(y, np_rms(x, w).astype(np.float16), max_ulp=1, what="fp16 rmsnorm")


def test_scale_invariance():
    r = tu.rng(35)
    x = tu.normal(r, (4, 4096), 0.0, 1.0, np.float32)
    w = tu.normal(r, (4096,), 1.0, 0.05, np.float32)
    y1 = oracle.rmsnorm_rows(x, w, 0.0)
    y2 = oracle.rmsnorm_rows(x * np.float32(8.0), w, 0.0)  # power of two: exact scaling
    tu.assert_f32_close(y2, y1, rel=1e-6, floor=1e-6)


def test_fused_equals_add_then_norm():
    r = tu.rng(36)
    for dt in (np.float16, np.float32):
        res = tu.normal(r, (32, 4096), dtype=dt)
        dx = tu.normal(r, (32, 4096), dtype=dt)
        w = tu.normal(r, (4096,), 1.0, 0.05, dt)
        new_res, y = oracle.residual_rmsnorm_rows(res, dx, w, EPS)
        added = oracle.residual_add(res, dx)
        assert tu.bits_equal(new_res, added)
        assert tu.bits_equal(y, oracle.rmsnorm_rows(added, w, EPS))
        # the fp16 residual is exactly one rounding of the fp32 sum
        expect = (res.astype(np.float32) + dx.astype(np.float32)).astype(dt)
        assert tu.bits_equal(added, expect)


def _round_f32(fr):
    """Exact rational -> nearest float32 (ties to even)."""
    from fractions import Fraction

    f = np.float32(float(fr))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                     int(np.float32(c).view(np.uint32)) & 1))


def test_reference_order_sum_known_answers():
    """oracle.ref_order_sumsq restates the reference kernel's fp32 order for
    sum(x^2) (cuda/rmsnorm_kernel.cu:16-22, cuda/cuda_utils.cuh:18-64).
    Hand-worked inputs where that order rounds differently from a sequential
    fp32 sum and from the exact sum pin the thread count, the per-thread fma
    and both shfl_down trees."""
    from fractions import Fraction

    # 1. n = 64, zero except x[25] = 3, x[40] = 2, x[46] = 1, x[54] = x[57] =
    # 6144 (squares 9, 4, 1, 37748736, 37748736): 64 threads, one element
    # each.  Warp 0 holds only 9.  Warp 1 (lanes 8, 14, 22, 25 = 4, 1, S, S
    # with S = 37748736, whose fp32 ulp is 4): offset 16 moves S to lanes 6
    # and 9; offset 8 gives lane 0 = 4, lane 1 = S, lane 6 = S + 1 -> S;
    # offset 4 moves S to lane 2; offset 2 gives lane 0 = S + 4 (exact);
    # offset 1: 2S + 4 = 75497476, a tie between 75497472 and 75497480 (ulp
    # 8), to even: 75497472.  The tree over the two warp sums: 9 + 75497472
    # -> 75497480.  A 32-thread split, an adjacent-pair tree, a sequential
    # fp32 sum and the exact sum (75497486) all give 75497488.
    x = np.zeros(64, np.float32)
    x[[25, 40, 46, 54, 57]] = [3.0, 2.0, 1.0, 6144.0, 6144.0]
    assert oracle.ref_order_sumsq(x) == np.float32(75497480.0)
    # 2. n = 2048: T = 1024 threads, thread 0 accumulates x[0]^2 then
    # x[1024]^2 as fma(v, v, acc) (nvcc contracts acc += v * v); every other
    # element is zero, so the trees pass thread 0's partial through.  For
    # these two values the contracted sum fl32(x1^2 + fl32(x0^2)) and the
    # separately rounded fl32(fl32(x1^2) + fl32(x0^2)) differ by one ulp.
    x = np.zeros(2048, np.float32)
    x0, x1 = np.float32(float.fromhex("0x1.e5ce34p+0")), np.float32(float.fromhex("0x1.d81f86p+0"))
    x[0], x[1024] = x0, x1
    a0 = _round_f32(Fraction(float(x0)) ** 2)
    fused = _round_f32(Fraction(float(x1)) ** 2 + Fraction(float(a0)))
    separate = _round_f32(Fraction(float(_round_f32(Fraction(float(x1)) ** 2))) +
                          Fraction(float(a0)))
    assert fused == np.float32(float.fromhex("0x1.c026cep+2")) and separate != fused
    assert oracle.ref_order_sumsq(x) == fused
    # 3. the config-1 row: the reference's rounding of sum(x^2) sits within
    # 1e-6 of the fp64 sum the oracle (and the GPU) use
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    x = g["rms1_x"][0]
    s32 = oracle.ref_order_sumsq(x)
    s64 = float(np.sum(x.astype(np.float64) ** 2))
    assert abs(s32 - s64) / s64 < 1e-6


def test_config1_fixture_reproduces_bit_for_bit():
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    y = oracle.rmsnorm_rows(g["rms1_x"], g["rms1_w"], EPS)
    assert tu.bits_equal(y, g["rms1_y"])
    for threads in (1, 4):
        oracle.set_threads(threads)
        assert tu.bits_equal(oracle.rmsnorm_rows(g["rms1_x"], g["rms1_w"], EPS), g["rms1_y"])
    oracle.set_threads(1)
