"""GPU parity: Q4_0 dequant-GEMV (jinf_cuda_dequant_matvec / jinf_matvec_q4_0)
against the oracle's fp64 dot product of the exactly dequantized matrix.

Bar: |y - y_oracle| <= 1e-5 * sum_j |w_j x_j| per row: the dot product's own
fp32 rounding scale (a relative bound on y itself is meaningless where the
terms cancel)."""
import ctypes

import numpy as np
import pytest
import torch

import jinf_amd
import oracle
import testutil as tu
from gpu_util import dev as to_dev
from gpu_util import host, say

pytestmark = pytest.mark.gpu


def check(y, ref, a, what):
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    worst = float(np.max(err / np.maximum(a, 1e-30)))
    say(f"{what}: worst error / sum|w x| = {worst:.2e}")
    assert worst <= 1e-5, what


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1024, 4096), (14336, 4096),
                                       (4096, 14336), (20000, 4096), (7, 128), (1, 64),
                                       (3, 2048), (515, 8192), (1024, 28672), (33, 32768)])
def test_llama_shapes(dev, rows, cols):
    say(f"matvec rows={rows} cols={cols}")
    r = tu.rng(rows + cols)
    W = tu.q4_0_table(r, rows, cols)
    x = tu.normal(r, (cols,), 0.0, 1.0, np.float32)
    oracle.set_threads(8)
    ref, a = oracle.matvec_q4_0(W, x)
    oracle.set_threads(1)
    y = host(jinf_amd.matvec_q4_0(to_dev(W), to_dev(x)))
    check(y, ref, a, f"{rows}x{cols}")


@pytest.mark.parametrize("rows,cols,w_off,x_off", [(33, 96, 0, 0), (50, 32 * 5, 0, 0),
                                                   (40, 4096, 2, 0), (40, 4096, 0, 1),
                                                   (17, 4160, 0, 0)])
def test_generic_path_and_drop_in(dev, rows, cols, w_off, x_off):
    say(f"drop-in matvec rows={rows} cols={cols} W+{w_off}B x+{x_off} floats")
    r = tu.rng(cols + w_off)
    W = tu.q4_0_table(r, rows, cols)
    x = tu.normal(r, (cols,), 0.0, 1.0, np.float32)
    ref, a = oracle.matvec_q4_0(W, x)
    wraw = np.zeros(W.size + 8, np.uint8)
    wraw[w_off:w_off + W.size] = W.reshape(-1)
    xraw = np.zeros(cols + 4, np.float32)
    xraw[x_off:x_off + cols] = x
    wd, xd = to_dev(wraw), to_dev(xraw)
    y = torch.full((rows + 1,), -7.0, dtype=torch.float32, device=dev)
    jinf_amd.lib().jinf_cuda_dequant_matvec(
        ctypes.c_void_p(wd.data_ptr() + w_off), ctypes.c_void_p(xd.data_ptr() + 4 * x_off),
        ctypes.c_void_p(y.data_ptr()), rows, cols, 2,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    yh = host(y)
    check(yh[:rows], ref, a, "drop-in")
    assert yh[rows] == -7.0


def test_one_hot_columns_exact(dev):
    say("one-hot x reproduces dequantized columns bit for bit")
    r = tu.rng(5)
    rows, cols = 256, 4096
    W = tu.q4_0_table(r, rows, cols)
    Wf = oracle.dequant_q4_0(W).reshape(rows, cols)
    wd = to_dev(W)
    for j in (0, 1, 30, 31, 32, 2047, 4095):
        x = np.zeros(cols, np.float32)
        x[j] = 1.0
        y = host(jinf_amd.matvec_q4_0(wd, to_dev(x)))
        assert tu.bits_equal(y, Wf[:, j]), j


def test_unsupported_qtype_leaves_output(dev):
    y = torch.full((16,), 3.0, dtype=torch.float32, device=dev)
    w = torch.zeros(16 * 144 // 1, dtype=torch.uint8, device=dev)
    x = torch.ones(256, dtype=torch.float32, device=dev)
    jinf_amd.cuda_dequant_matvec(w, x, y, 16, 256, qtype=12)
    assert np.all(host(y) == 3.0)
