"""Pins the oracle's masked row softmax (cuda/softmax_kernel.cu:8-42, the
attention softmax phase cuda/attention_kernel.cu:59-87).

Pinned by scipy.special.softmax in float64, normalisation (sum = 1), shift
invariance, closed forms (length-1 row -> 1.0, uniform row -> 1/n, one huge
logit -> 1), the scale applied before the max, and the masked tail left
untouched (poisoned with NaN).
"""
import numpy as np
from scipy.special import softmax as sp_softmax

import oracle
import testutil as tu

# The reference forms s - m in fp32: with |s - m| up to ~30 that rounding alone
# moves exp(s - m) by up to 30 * 2^-24 ~ 1.8e-6 relative; three more roundings
# (exp, 1/sum, product) add < 2e-7.  Against exact float64 softmax: 2.5e-6.
REL = 2.5e-6


def test_vs_scipy():
    r = tu.rng(61)
    x = tu.normal(r, (64, 3000), 0.0, 3.0, np.float32)
    y = oracle.softmax_rows(x)
    tu.assert_f32_close(y, sp_softmax(x.astype(np.float64), axis=1), rel=REL, floor=1e-30)
    assert np.max(np.abs(y.astype(np.float64).sum(axis=1) - 1)) < 1e-5


def test_masked_lengths_and_tail_untouched():
    r = tu.rng(62)
    x = tu.normal(r, (6, 512), 0.0, 3.0, np.float32)
    lens = np.array([1, 7, 512, 600, 0, -3], np.int32)
    poison = np.full_like(x, np.nan)
    y = oracle.softmax_rows(x, lens, 1, 1.0, out=poison)
    for i, L in enumerate([1, 7, 512, 512, 0, 0]):
        assert np.all(np.isnan(y[i, L:]))
        if L:
            tu.assert_f32_close(y[i, :L], sp_softmax(x[i, :L].astype(np.float64)), rel=REL)
    assert y[0, 0] == 1.0


def test_rows_per_len_and_scale():
    r = tu.rng(63)
    x = tu.normal(r, (8, 256), 0.0, 1.0, np.float32)
    lens = np.array([100, 256], np.int32)
    y = oracle.softmax_rows(x, lens, 4, 0.125, out=np.zeros_like(x))
    for i in range(8):
        L = lens[i // 4]
        ref = sp_softmax(0.125 * x[i, :L].astype(np.float64))
        tu.assert_f32_close(y[i, :L], ref, rel=REL)
        assert np.all(y[i, L:] == 0)


def test_closed_forms_and_shift():
    n = 1000
    y = oracle.softmax_rows(np.full((1, n), 2.5, np.float32))
    assert np.all(y == np.float32(1.0) / np.float32(n))
    x = np.zeros((1, n), np.float32)
    x[0, 3] = 200.0
    y = oracle.softmax_rows(x)
    assert y[0, 3] == 1.0 and np.all(np.delete(y[0], 3) == 0)
    r = tu.rng(64)
    x = tu.normal(r, (4, 777), 0.0, 3.0, np.float32)
    tu.assert_f32_close(oracle.softmax_rows(x + np.float32(16.0)), oracle.softmax_rows(x),
                        rel=1e-5, floor=1e-30)
