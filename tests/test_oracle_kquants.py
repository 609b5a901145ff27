"""Pins the oracle's Q8_0, Q4_K and Q6_K dequantization and its generic GEMV
(src/quant.cpp:64-105, cuda/dequant_kernels.cu:25-110,
cuda/matmul_kernels.cu:47-185).

Pinned by:
- Q4_K and Q8_0: the reference's own CPU routines (jinf_dequantize_q4_K /
  _q8_0, compiled from src/quant.cpp into oracle/_ref), bit for bit, on random
  blocks and on every byte value of the scale array; the frozen outputs are in
  tests/golden/kquants_ref.npz for hosts without oracle/_ref;
- Q6_K (the reference has no CPU routine): known answers derived by hand from
  the element mapping of cuda/dequant_kernels.cu:97-106 (ql nibble by element
  parity, qh two-bit field 2*(e%4), scale e/16, d stored last), chosen so that
  a swapped nibble, a wrong qh shift, a wrong scale index, an unsigned scale or
  d read from the front of the block each fail;
- the GEMV: numpy's float64 product of the dequantized matrix (an
  independent BLAS routine) and a one-hot x selecting a column exactly.
"""
import os

import numpy as np
import pytest

import oracle
import testutil as tu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kquants_ref.npz")


def test_geometry():
    assert oracle.qtype_geometry(oracle.Q4_0) == (32, 18)
    assert oracle.qtype_geometry(oracle.Q8_0) == (32, 34)
    assert oracle.qtype_geometry(oracle.Q4_K) == (256, 144)
    assert oracle.qtype_geometry(oracle.Q6_K) == (256, 210)
    assert oracle.qtype_geometry(3) == (0, 0)


@pytest.mark.parametrize("qtype", [oracle.Q4_K, oracle.Q8_0])
def test_matches_reference_cpu_routine(qtype):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (the golden test below covers this host)")
    r = tu.rng(qtype)
    e, nbytes = oracle.qtype_geometry(qtype)
    W = tu.quant_table(r, qtype, 1, e * 64, 0.05)
    assert tu.bits_equal(oracle.dequant(qtype, W), oracle.ref_dequant(qtype, W))


def test_matches_frozen_reference_outputs():
    g = np.load(GOLDEN)
    for qtype, key in ((oracle.Q4_K, "q4_K"), (oracle.Q8_0, "q8_0")):
        got = oracle.dequant(qtype, g[key + "_blocks"])
        assert tu.bits_equal(got, g[key + "_out"]), key


def test_q4_K_scale_unpacking_every_byte():
    """All 256 values in every scale byte position: a sub-block's output
    reveals its (sc, mn) pair with d = dmin = 1 and q = 0 / 1."""
    blocks = []
    for pos in range(12):
        for v in range(256):
            b = np.zeros(144, np.uint8)
            b[0:2] = np.array([1.0], np.float16).view(np.uint8)
            b[2:4] = np.array([1.0], np.float16).view(np.uint8)
            b[4 + pos] = v
            b[16:] = 0x10  # element 2i: q = 0, element 2i+1: q = 1
            blocks.append(b)
    out = oracle.dequant(oracle.Q4_K, np.concatenate(blocks)).reshape(-1, 8, 32)
    mn = -out[:, :, 0]
    sc = out[:, :, 1] + mn
    # the reference's unpacking (src/quant.cpp:70-75), element by element
    k = 0
    for pos in range(12):
        for v in range(256):
            s = np.zeros(12, np.int64)
            s[pos] = v
            exp_sc = [s[i] & 63 for i in range(4)] + [((s[i + 8] & 15) << 2) | (s[i] >> 6) for i in range(4)]
            exp_mn = [s[i + 4] & 63 for i in range(4)] + [((s[i + 8] >> 4) << 2) | (s[i + 4] >> 6) for i in range(4)]
            assert list(sc[k]) == exp_sc and list(mn[k]) == exp_mn, (pos, v)
            k += 1


def _q6_block(d=1.0):
    b = np.zeros(210, np.uint8)
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    b[192:208] = 1  # every sub-block scale = 1
    return b


def test_q6_K_known_answers():
    # all-zero bits: q6 = 0 -> -32 * d * scale
    b = _q6_block(0.5)
    assert np.all(oracle.dequant(oracle.Q6_K, b) == -16.0)
    # ql[0] = 0x21: element 0 low nibble 1, element 1 high nibble 2
    # qh[0] = 0b11_10_01_00: elements 0..3 get high bits 0, 1, 2, 3
    b = _q6_block()
    b[0] = 0x21
    b[1] = 0x43  # element 2: 3, element 3: 4
    b[128] = 0b11100100
    out = oracle.dequant(oracle.Q6_K, b)
    assert list(out[:4]) == [1 - 32, (2 | 16) - 32, (3 | 32) - 32, (4 | 48) - 32]
    assert np.all(out[4:] == -32.0)
    # element 255: ql[127] high nibble, qh[63] bits 6-7, scale[15]
    b = _q6_block()
    b[127] = 0xF0
    b[191] = 0xC0
    b[207] = 0xFE  # int8 -2
    out = oracle.dequant(oracle.Q6_K, b)
    assert out[255] == -2.0 * (63 - 32)
    assert out[254] == -2.0 * (0 - 32)          # same scale (sub-block 15), bits clear
    assert np.all(out[240:254] == 64.0)
    assert np.all(out[:240] == -32.0)
    # sub-block scale index e / 16 and d at the end of the block
    b = _q6_block(2.0)
    b[192 + 3] = 5
    out = oracle.dequant(oracle.Q6_K, b)
    assert np.all(out[48:64] == 2.0 * 5 * -32) and np.all(out[:48] == -64.0)


def test_q8_0_known_answers():
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([0.25], np.float16).view(np.uint8)
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert list(oracle.dequant(oracle.Q8_0, b)) == [0.25 * v for v in range(-16, 16)]


@pytest.mark.parametrize("qtype", [oracle.Q4_0, oracle.Q8_0, oracle.Q4_K, oracle.Q6_K])
def test_matvec_vs_numpy_dot(qtype):
    r = tu.rng(80 + qtype)
    for rows, cols in ((32, 4096), (5, 2048)):
        W = tu.quant_table(r, qtype, rows, cols)
        x = tu.normal(r, (cols,), 0.0, 1.0, np.float32)
        y, a = oracle.matvec(qtype, W, x)
        Wf = oracle.dequant(qtype, W).reshape(rows, cols).astype(np.float64)
        ref = Wf @ x.astype(np.float64)
        assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-7 * a + 1e-30)
        assert np.allclose(a, np.abs(Wf) @ np.abs(x.astype(np.float64)), rtol=1e-12)
        if qtype == oracle.Q4_0:
            assert tu.bits_equal(y, oracle.matvec_q4_0(W, x)[0])


@pytest.mark.parametrize("qtype", [oracle.Q8_0, oracle.Q4_K, oracle.Q6_K])
def test_matvec_one_hot_selects_a_column(qtype):
    r = tu.rng(90 + qtype)
    rows, cols = 8, 512
    W = tu.quant_table(r, qtype, rows, cols)
    Wf = oracle.dequant(qtype, W).reshape(rows, cols)
    for j in (0, 1, 17, 255, 256, 511):
        x = np.zeros(cols, np.float32)
        x[j] = 1.0
        assert tu.bits_equal(oracle.matvec(qtype, W, x)[0], Wf[:, j])
