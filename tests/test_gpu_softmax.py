"""GPU parity: masked fp32 row softmax (attention-score rows) and the
single-row drop-in.

Bar: within 1e-5 relative of the oracle (floor 1e-30 for values that underflow
towards fp32 subnormals), masked tails never written (poisoned with NaN), rows
sum to 1 at the full config-5 size.
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


def test_config5_ragged_rows(dev):
    say("config 5: 64 seqs x 64 heads, stride 8192, len = pos + 1, logits ~ N(0, 3)")
    r = tu.rng(5)
    pos = r.integers(0, 8192, size=64)
    lens = (pos + 1).astype(np.int32)
    x = tu.normal(r, (4096, 8192), 0.0, 3.0, np.float32)
    oracle.set_threads(8)
    ref = oracle.softmax_rows(x, lens, 64, 1.0, out=np.full_like(x, np.nan))
    oracle.set_threads(1)
    xd = to_dev(x)
    out = torch.full_like(xd, float("nan"))
    jinf_amd.softmax_rows(xd, to_dev(lens), 64, 1.0, out=out)
    got = host(out)
    live = ~np.isnan(ref)
    assert np.array_equal(np.isnan(got), ~live)  # tails untouched
    tu.assert_f32_close(got[live], ref[live], 1e-5, 1e-30, "config 5")
    sums = np.nansum(got.astype(np.float64), axis=1)
    assert np.max(np.abs(sums - 1.0)) < 1e-5
    assert tu.bits_equal(host(xd), x)  # input untouched


def test_wide_exponent_range(dev):
    # s - m spread evenly over [-87, 0]: every normal fp32 result, down to
    # about 1.6e-38, where the two-operation exponential's error bound
    # (7.3e-8 |a| + 1.2e-7 relative) is largest; offsets move the maxima
    say("exponent range: s - m over [-87, 0], maxima at 0, 40, -30, 1000")
    r = tu.rng(91)
    n = 8192
    base = np.linspace(-87.0, 0.0, n)
    x = np.stack([(r.permutation(base) + off).astype(np.float32)
                  for off in (0.0, 40.0, -30.0, 1000.0)])
    lens = np.full(4, n, np.int32)
    ref = oracle.softmax_rows(x, lens, 1, 1.0, out=np.full_like(x, np.nan))
    xd = to_dev(x)
    out = torch.full_like(xd, float("nan"))
    jinf_amd.softmax_rows(xd, to_dev(lens), 1, 1.0, out=out)
    got = host(out)
    tu.assert_f32_close(got, ref, 1e-5, 1e-30, "wide range")
    exact = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True).astype(np.float64))
    exact /= exact.sum(axis=1, keepdims=True)
    big = exact >= 1e-30
    err = np.max(np.abs(got[big] - exact[big]) / exact[big])
    say(f"max relative error against fp64 over results >= 1e-30: {err:.2e}")
    assert err < 1e-5


def test_fixture(dev):
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    xd = to_dev(g["sm_x"])
    out = torch.full_like(xd, float("nan"))
    jinf_amd.softmax_rows(xd, to_dev(g["sm_lens"]), 4, 1.0, out=out)
    got, ref = host(out), g["sm_y"]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    live = ~np.isnan(ref)
    tu.assert_f32_close(got[live], ref[live], 1e-5, 1e-30, "fixture")


@pytest.mark.parametrize("n", [1, 3, 100, 1024, 8192, 32768, 40000, 100003])
def test_drop_in_single_row(dev, n):
    say(f"drop-in jinf_cuda_softmax n={n} (in place)")
    r = tu.rng(n)
    x = tu.normal(r, (1, n), 0.0, 3.0, np.float32)
    ref = oracle.softmax_rows(x)
    xd = to_dev(x[0])
    jinf_amd.cuda_softmax(xd, xd)
    tu.assert_f32_close(host(xd), ref[0], 1e-5, 1e-30, f"n={n}")


def test_scale_lengths_and_unaligned_rows(dev):
    say("scale 1/sqrt(128), per-row lens incl. 0 and > n, row stride 1001")
    r = tu.rng(77)
    x = tu.normal(r, (40, 1001), 0.0, 3.0, np.float32)
    lens = r.integers(-3, 1100, size=40).astype(np.int32)
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    ref = oracle.softmax_rows(x, lens, 1, scale, out=np.full_like(x, np.nan))
    xd = to_dev(x)
    out = torch.full_like(xd, float("nan"))
    jinf_amd.softmax_rows(xd, to_dev(lens), 1, scale, out=out)
    got = host(out)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    live = ~np.isnan(ref)
    tu.assert_f32_close(got[live], ref[live], 1e-5, 1e-30, "scaled")


def test_all_masked_rows_noop_and_length_one(dev):
    x = np.random.default_rng(3).normal(0, 3, size=(4, 64)).astype(np.float32)
    lens = np.array([0, 1, 1, 0], np.int32)
    xd = to_dev(x)
    out = torch.full_like(xd, 7.0)
    jinf_amd.softmax_rows(xd, to_dev(lens), 1, 1.0, out=out)
    got = host(out)
    assert np.all(got[0] == 7.0) and np.all(got[3] == 7.0)
    assert got[1, 0] == 1.0 and got[2, 0] == 1.0 and np.all(got[1:3, 1:] == 7.0)


@pytest.mark.parametrize("n_rows,rows_per_len,n_cols", [
    (70, 8, 4096),       # last length entry covers 6 rows only
    (5, 100, 512),       # one entry, more rows per entry than rows
    (65537, 1, 64),      # more entries than a grid dimension holds: 1-D grid
    (12, 3, 16384),      # 1024 lanes x 4 chunks
    (6, 2, 256),         # 64 lanes
    (9, 9, 20000),       # 1024 lanes x 8 chunks, length entries past 16384
])
def test_grid_shapes(dev, n_rows, rows_per_len, n_cols):
    say(f"{n_rows} rows, {rows_per_len} rows per length, {n_cols} columns")
    r = tu.rng(n_rows + n_cols)
    x = tu.normal(r, (n_rows, n_cols), 0.0, 3.0, np.float32)
    n_len = -(-n_rows // rows_per_len)
    lens = r.integers(0, n_cols + 2, size=n_len).astype(np.int32)
    lens[0] = n_cols
    ref = oracle.softmax_rows(x, lens, rows_per_len, 1.0, out=np.full_like(x, np.nan))
    xd = to_dev(x)
    out = torch.full_like(xd, float("nan"))
    jinf_amd.softmax_rows(xd, to_dev(lens), rows_per_len, 1.0, out=out)
    got = host(out)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    live = ~np.isnan(ref)
    tu.assert_f32_close(got[live], ref[live], 1e-5, 1e-30, "grid shapes")
