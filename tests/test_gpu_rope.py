"""GPU parity: interleaved RoPE (drop-in fp32 and fp16/fp32 rows).

Bar: fp16 within 2 ulp of the oracle; fp32 within 1e-5 of |ref| per element
(north_star's tolerance).  The GPU evaluates (cos, sin) in fp64 from the same
fp32 angle, rounds them once to fp32 and applies the rotation without
contraction, like the oracle, so the outputs are expected to be bit-identical;
each test reports the bit-identical fraction.  The relative error of an output
near zero is also reported against max(|ref|, |pair|): such an output is a
difference of two products, so a 1-ulp difference in cos or sin would show
up there first.
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


def pair_floor(x, hd):
    """Per-element |pair| of the input, for the fp32 relative bound."""
    x = x.astype(np.float64).reshape(x.shape[0], -1, 2)
    n = np.hypot(x[..., 0], x[..., 1])
    return np.repeat(n, 2, axis=-1).reshape(x.shape[0], -1)


def check(got, ref, src, hd, what):
    if got.dtype == np.float16:
        w = tu.assert_f16_close(got, ref, 2, what)
    else:
        w = tu.assert_f32_close(got, ref, 1e-5, 1e-30, what)
        err = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)),
                                                                 pair_floor(src, hd))
        say(f"{what}: worst error relative to the pair norm {float(err.max()):.3g}")
    exact = float(np.mean(got.view(np.uint16 if got.dtype == np.float16 else np.uint32)
                          == ref.view(np.uint16 if ref.dtype == np.float16 else np.uint32)))
    say(f"{what}: worst {w}, bit-identical fraction {exact:.6f}")
    return exact


def test_config2_full(dev):
    say("config 2: Q [512,32,128] K [512,8,128] fp16, pos 0..511, theta 500000")
    r = tu.rng(2)
    q = tu.normal(r, (512, 32 * 128))
    k = tu.normal(r, (512, 8 * 128))
    pos = np.arange(512, dtype=np.int32)
    rq, rk = oracle.rope_rows(q, k, 128, pos, 0, 500000.0)
    qd, kd = to_dev(q), to_dev(k)
    jinf_amd.rope_rows(qd, kd, 128, to_dev(pos), 0, 500000.0)
    # observed bit-identical: (cos, sin) are the correctly rounded values on
    # both sides and the rotation rounds at the same points
    assert check(host(qd), rq, q, 128, "q") == 1.0
    assert check(host(kd), rk, k, 128, "k") == 1.0


def test_config5_decode_shape(dev):
    say("70B decode: Q [64, 64*128] K [64, 8*128], pos ~ U[0, 8192)")
    r = tu.rng(55)
    q = tu.normal(r, (64, 64 * 128))
    k = tu.normal(r, (64, 8 * 128))
    pos = r.integers(0, 8192, size=64).astype(np.int32)
    rq, rk = oracle.rope_rows(q, k, 128, pos, 0, 500000.0)
    qd, kd = to_dev(q), to_dev(k)
    jinf_amd.rope_rows(qd, kd, 128, to_dev(pos), 0, 500000.0)
    assert check(host(qd), rq, q, 128, "q") == 1.0
    assert check(host(kd), rk, k, 128, "k") == 1.0


def test_fixture(dev):
    say("committed RoPE fixture")
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    qd, kd = to_dev(g["rope_q"]), to_dev(g["rope_k"])
    jinf_amd.rope_rows(qd, kd, 128, to_dev(g["rope_pos"]), 0, 500000.0)
    tu.assert_f16_close(host(qd), g["rope_q_out"], 2, "q")
    tu.assert_f16_close(host(kd), g["rope_k_out"], 2, "k")


@pytest.mark.parametrize("pos", [0, 1, 511, 8191])
@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_drop_in_single_token(dev, pos, base):
    say(f"drop-in jinf_cuda_rope pos={pos} base={base}")
    r = tu.rng(pos + 3)
    q = tu.normal(r, (1, 32 * 128), dtype=np.float32)
    k = tu.normal(r, (1, 8 * 128), dtype=np.float32)
    rq, rk = oracle.rope_rows(q, k, 128, None, pos, base)
    qd, kd = to_dev(q[0]), to_dev(k[0])
    jinf_amd.cuda_rope(qd, kd, 128, 32, 8, pos, base)
    check(host(qd)[None], rq, q, 128, "q")
    check(host(kd)[None], rk, k, 128, "k")
    if pos == 0:
        assert tu.bits_equal(host(qd), q[0]) and tu.bits_equal(host(kd), k[0])


@pytest.mark.parametrize("hd,nh,nkv,ldpad", [(6, 3, 1, 0), (128, 4, 2, 2), (64, 2, 2, 0),
                                             (512, 2, 1, 0), (2, 5, 5, 0)])
@pytest.mark.parametrize("dt", [np.float16, np.float32])
def test_shapes_and_scalar_path(dev, hd, nh, nkv, ldpad, dt):
    say(f"head_dim={hd} heads {nh}/{nkv} ld pad {ldpad} {np.dtype(dt).name}")
    r = tu.rng(hd + nh)
    T = 9
    qb = tu.normal(r, (T, nh * hd + ldpad), dtype=dt)
    kb = tu.normal(r, (T, nkv * hd + ldpad), dtype=dt)
    pos = r.integers(0, 8192, size=T).astype(np.int32)
    q = np.ascontiguousarray(qb[:, :nh * hd])
    k = np.ascontiguousarray(kb[:, :nkv * hd])
    rq, rk = oracle.rope_rows(q, k, hd, pos, 0, 10000.0)
    qd, kd = to_dev(qb), to_dev(kb)
    jinf_amd.rope_rows(qd[:, :nh * hd], kd[:, :nkv * hd], hd, to_dev(pos), 0, 10000.0)
    gq, gk = host(qd), host(kd)
    check(np.ascontiguousarray(gq[:, :nh * hd]), rq, q, hd, "q")
    check(np.ascontiguousarray(gk[:, :nkv * hd]), rk, k, hd, "k")
    assert tu.bits_equal(gq[:, nh * hd:], qb[:, nh * hd:])  # padding untouched
    assert tu.bits_equal(gk[:, nkv * hd:], kb[:, nkv * hd:])


def test_full_size_norm_preservation(dev):
    say("config 2 size, fp32: pair norms preserved")
    r = tu.rng(56)
    q = torch.from_numpy(tu.normal(r, (512, 32 * 128), dtype=np.float32)).to(dev)
    k = torch.from_numpy(tu.normal(r, (512, 8 * 128), dtype=np.float32)).to(dev)
    q0, k0 = q.clone(), k.clone()
    jinf_amd.rope_rows(q, k, 128, None, 0, 500000.0)
    for a, b in ((q0, q), (k0, k)):
        na = torch.hypot(a[:, 0::2].double(), a[:, 1::2].double())
        nb = torch.hypot(b[:, 0::2].double(), b[:, 1::2].double())
        assert float(((nb - na).abs() / na.clamp_min(1e-30)).max()) < 1e-6


@pytest.mark.parametrize("hd", [128, 64, 256])
def test_large_positions_fp32(dev, hd):
    """Positions up to 2^31 - 1: angles beyond 2^20 take the device library's
    fp64 sincos, smaller ones the library's own reduction; pair 0 (theta = 1)
    rotates by the position itself.  Every output within 1e-5 per element."""
    say(f"fp32 rows, head_dim {hd}, positions up to 2^31 - 1")
    r = tu.rng(hd + 7)
    pos = np.array([0, 1, 2, 3, 4, 1000, 8191, 65535, 102943, 1 << 20, (1 << 20) - 1,
                    (1 << 20) + 1, 1647099, 1647100, 16777215, 16777217, 123456789,
                    (1 << 31) - 1, 1 << 30, 355, 710, 1068966896], np.int32)
    T = pos.size
    q = tu.normal(r, (T, 4 * hd), dtype=np.float32)
    k = tu.normal(r, (T, 2 * hd), dtype=np.float32)
    for base in (10000.0, 500000.0):
        rq, rk = oracle.rope_rows(q, k, hd, pos, 0, base)
        qd, kd = to_dev(q), to_dev(k)
        jinf_amd.rope_rows(qd, kd, hd, to_dev(pos), 0, base)
        check(host(qd), rq, q, hd, f"q base {base:g}")
        check(host(kd), rk, k, hd, f"k base {base:g}")
