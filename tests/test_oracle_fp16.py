"""Pins the oracle's binary16 <-> binary32 conversions.

Checked against numpy's IEEE conversions (an independent implementation) on
every binary16 pattern and on the fp32 values where rounding is decided (ties,
one ulp either side of ties, overflow and underflow thresholds), and against
the reference's own fp16_to_fp32 (src/quant.cpp:7-45) via the golden fixture
written from the compiled reference.
"""
import os

import numpy as np
import pytest

import oracle
import testutil as tu

HERE = os.path.dirname(os.path.abspath(__file__))


def all_f16():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)


def test_f16_to_f32_exhaustive_vs_numpy():
    h = all_f16()
    assert tu.bits_equal(oracle.f16_to_f32(h), h.astype(np.float32))


def test_f16_to_f32_exhaustive_vs_reference_fixture():
    g = np.load(os.path.join(HERE, "golden", "q4_0_ref.npz"))
    h = g["f16_bits"].view(np.float16)
    got = oracle.f16_to_f32(h)
    # bit-exact including NaN payloads: the reference shifts the mantissa up
    assert np.array_equal(got.view(np.uint32), g["f16_to_f32"].view(np.uint32))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
def test_f16_to_f32_vs_reference_library():
    h = all_f16()
    assert np.array_equal(oracle.f16_to_f32(h).view(np.uint32),
                          oracle.ref_f16_to_f32(h).view(np.uint32))


def test_f32_to_f16_round_trip_exhaustive():
    h = all_f16()
    back = oracle.f32_to_f16(h.astype(np.float32))
    assert tu.bits_equal(back, h)


def test_f32_to_f16_ties_and_neighbours_vs_numpy():
    h = all_f16()
    f = h.astype(np.float64)
    ok = np.isfinite(f)
    f = f[ok]
    with np.errstate(over="ignore"):
        nxt = np.nextafter(h[ok], np.float16(np.inf)).astype(np.float64)
    fin = np.isfinite(nxt)
    mid = ((f[fin] + nxt[fin]) / 2).astype(np.float32)  # exact in fp32: ties
    cand = np.concatenate([
        mid,
        np.nextafter(mid, np.float32(np.inf)),
        np.nextafter(mid, np.float32(-np.inf)),
    ])
    assert tu.bits_equal(oracle.f32_to_f16(cand), cand.astype(np.float16))


def test_f32_to_f16_thresholds_vs_numpy():
    vals = np.array([
        65504.0, 65519.996, 65520.0, 65536.0, 1e30, np.inf, -np.inf, np.nan,
        2.0 ** -14, 2.0 ** -15, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
        2.0 ** -24 * 1.5, 2.0 ** -24 * 2.5, 2.0 ** -26, 1e-45, 0.0, -0.0,
        -2.0 ** -25, -2.0 ** -24 * 1.5, 6.1035156e-05, 6.0975552e-05,
    ], dtype=np.float32)
    vals = np.concatenate([vals, np.nextafter(vals, np.float32(np.inf)),
                           np.nextafter(vals, np.float32(-np.inf))])
    with np.errstate(over="ignore"):
        expect = vals.astype(np.float16)
    assert tu.bits_equal(oracle.f32_to_f16(vals), expect)


def test_f32_to_f16_random_vs_numpy():
    r = tu.rng(11)
    bits = r.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        expect = x.astype(np.float16)
    assert tu.bits_equal(oracle.f32_to_f16(x), expect)
