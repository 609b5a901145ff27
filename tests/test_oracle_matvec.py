"""Pins the oracle's Q4_0 dequant-GEMV (cuda/matmul_kernels.cu:8-43).

Pinned by: the oracle's own Q4_0 dequant (itself pinned to the reference's
compiled src/quant.cpp) followed by numpy's float64 matrix-vector product (an
independent BLAS routine); a one-hot x picks out one dequantized column
exactly; linearity in x; the interleaved element order (a swapped nibble order
fails the one-hot check)."""
import numpy as np

import oracle
import testutil as tu


def test_vs_numpy_dot_of_dequantized_matrix():
    r = tu.rng(71)
    for rows, cols in ((64, 4096), (33, 96), (5, 14336)):
        W = tu.q4_0_table(r, rows, cols)
        x = tu.normal(r, (cols,), 0.0, 1.0, np.float32)
        y, a = oracle.matvec_q4_0(W, x)
        Wf = oracle.dequant_q4_0(W).reshape(rows, cols).astype(np.float64)
        ref = Wf @ x.astype(np.float64)
        assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-7 * a + 1e-30)
        assert np.allclose(a, np.abs(Wf) @ np.abs(x.astype(np.float64)), rtol=1e-12)


def test_one_hot_selects_a_column():
    r = tu.rng(72)
    rows, cols = 16, 256
    W = tu.q4_0_table(r, rows, cols)
    Wf = oracle.dequant_q4_0(W).reshape(rows, cols)
    for j in (0, 1, 2, 31, 32, 33, 255):
        x = np.zeros(cols, np.float32)
        x[j] = 1.0
        y, _ = oracle.matvec_q4_0(W, x)
        assert tu.bits_equal(y, Wf[:, j])


def test_linearity():
    r = tu.rng(73)
    W = tu.q4_0_table(r, 8, 512)
    x1 = tu.normal(r, (512,), 0.0, 1.0, np.float32)
    x2 = tu.normal(r, (512,), 0.0, 1.0, np.float32)
    y1, a1 = oracle.matvec_q4_0(W, x1)
    y2, a2 = oracle.matvec_q4_0(W, x2)
    y12, _ = oracle.matvec_q4_0(W, (x1 + x2).astype(np.float32))
    assert np.all(np.abs(y12.astype(np.float64) - (y1.astype(np.float64) + y2)) <= 1e-6 * (a1 + a2))
