"""Pins the oracle's Q4_0 dequant / gather (src/quant.cpp:49-60,
cuda/dequant_kernels.cu:6-21, row addressing src/engine.cpp:170-178,311-317).

Pinned by: the reference's own compiled CPU dequantizer (golden fixture, and
the library itself when oracle/_ref is built), an independent numpy closed
form, and known answers for the interleaved element order and the special
scale classes (-0.0, Inf*0 = NaN, subnormal scales).
"""
import os

import numpy as np
import pytest

import oracle
import testutil as tu

HERE = os.path.dirname(os.path.abspath(__file__))


def numpy_dequant(blocks):
    """Closed form written independently with numpy float32 arithmetic."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)  # [n, 1]
    qs = b[:, 2:].astype(np.int32)
    lo = (qs & 15) - 8
    hi = (qs >> 4) - 8
    vals = np.stack([lo, hi], axis=2).reshape(-1, 32).astype(np.float32)  # interleaved
    with np.errstate(invalid="ignore"):
        return (vals * d).reshape(-1)


def test_matches_reference_fixture():
    g = np.load(os.path.join(HERE, "golden", "q4_0_ref.npz"))
    got = oracle.dequant_q4_0(g["blocks"])
    assert tu.bits_equal(got, g["out"])


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
def test_matches_reference_library_random():
    r = tu.rng(21)
    t = tu.q4_0_table(r, 512, 4096)
    # include wide-range scales too: random fp16 bit patterns
    t2 = t.copy().reshape(-1, 18)
    t2[::3, 0:2] = r.integers(0, 65536, size=(t2[::3].shape[0], 1), dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    for blocks in (t, t2):
        assert tu.bits_equal(oracle.dequant_q4_0(blocks), oracle.ref_dequant_q4_0(blocks))


def test_matches_numpy_closed_form():
    r = tu.rng(22)
    t = tu.q4_0_table(r, 64, 1024).reshape(-1, 18)
    t[::5, 0:2] = r.integers(0, 65536, size=(t[::5].shape[0], 1), dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    assert tu.bits_equal(oracle.dequant_q4_0(t), numpy_dequant(t))


def test_interleaved_order_known_answer():
    # qs[j] = 0x21: low nibble 1 -> element 2j = -7*d, high nibble 2 -> 2j+1 = -6*d
    qs = np.zeros((1, 16), np.uint8) + 0x88
    qs[0, 5] = 0x21
    out = oracle.dequant_q4_0(tu.q4_0_blocks([0x3C00], qs))  # d = 1.0
    expect = np.zeros(32, np.float32)
    expect[10], expect[11] = -7.0, -6.0
    assert tu.bits_equal(out, expect)  # the other nibbles are 8 -> +0.0


def test_special_scales():
    qs = np.arange(16, dtype=np.uint8)[None, :] * 17  # bytes 0x00, 0x11, ... 0xFF
    out = oracle.dequant_q4_0(tu.q4_0_blocks([0x0000], qs))  # d = +0
    nib = np.repeat(np.arange(16), 2)
    bits = out.view(np.uint32)
    assert np.all(bits[nib < 8] == 0x80000000)  # negative * +0 = -0.0
    assert np.all(bits[nib >= 8] == 0)
    out = oracle.dequant_q4_0(tu.q4_0_blocks([0x7C00], qs))  # d = +Inf
    assert np.all(np.isnan(out[nib == 8]))
    assert np.all(out[nib > 8] == np.inf) and np.all(out[nib < 8] == -np.inf)
    out = oracle.dequant_q4_0(tu.q4_0_blocks([0x0001], qs))  # smallest subnormal
    assert np.array_equal(out, (nib - 8).astype(np.float32) * np.float32(2.0 ** -24))
    out = oracle.dequant_q4_0(tu.q4_0_blocks([0x3C00], qs))  # d = 1: integers -8..7
    assert np.array_equal(out, (nib - 8).astype(np.float32))


def test_fp16_output_is_single_rounding_of_exact():
    r = tu.rng(23)
    t = tu.q4_0_table(r, 32, 512)
    t.reshape(-1, 18)[::2, 0:2] = r.integers(0, 65536, size=(t.size // 36, 1), dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    f32 = oracle.embed_q4_0(t, None, 512, np.float32)
    f16 = oracle.embed_q4_0(t, None, 512, np.float16)
    with np.errstate(over="ignore"):
        assert tu.bits_equal(f16, f32.astype(np.float16))


def test_gather_addressing_and_bad_ids():
    r = tu.rng(24)
    t = tu.q4_0_table(r, 100, 256)
    ids = np.array([5, 0, 99, 5, -1, 100, 42], np.int32)
    out = oracle.embed_q4_0(t, ids, 256, np.float32)
    for i, idx in enumerate(ids):
        if 0 <= idx < 100:
            assert tu.bits_equal(out[i], numpy_dequant(t[idx]))
        else:
            assert np.all(out[i].view(np.uint32) == 0)  # +0.0 rows
