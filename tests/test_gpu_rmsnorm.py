"""GPU parity: RMSNorm (drop-in and rows) and fused residual add + RMSNorm.

Bar: fp16 outputs within 2 ulp of the oracle, fp32 within 1e-5 relative, the
fp16 residual and the config-1 row bit-exact.  Both the GPU and the oracle sum
squares in fp64 and take 1/sqrt in fp64, so in practice they agree bit for
bit; the tolerance covers the last-bit cases where the two fp64 sums (in
different orders) round to different fp32 values.
"""
import ctypes
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
EPS = 1e-5


def test_config1_drop_in_bit_for_bit(dev):
    say("config 1: jinf_cuda_rmsnorm fp32 1x4096 vs committed fixture")
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    x, w, y = g["rms1_x"][0], g["rms1_w"], g["rms1_y"][0]
    out = torch.empty(4096, dtype=torch.float32, device=dev)
    jinf_amd.cuda_rmsnorm(out, to_dev(x), to_dev(w), EPS)
    assert tu.bits_equal(host(out), y)


@pytest.mark.parametrize("n", [1, 63, 64, 1000, 4096, 8192, 16384, 40000])
@pytest.mark.parametrize("wdt", [np.float32, np.float16])
def test_drop_in_sizes_in_place(dev, n, wdt):
    say(f"drop-in rmsnorm n={n} weight {np.dtype(wdt).name} in place")
    r = tu.rng(100 + n)
    x = tu.normal(r, (1, n), 0.0, 1.0, np.float32)
    w = tu.normal(r, (n,), 1.0, 0.05, wdt)
    ref = oracle.rmsnorm_rows(x, w, EPS)[0]
    buf = to_dev(x[0])
    jinf_amd.cuda_rmsnorm(buf, buf, to_dev(w), EPS)
    tu.assert_f32_close(host(buf), ref, rel=1e-5, floor=1e-30, what=f"n={n}")


def test_config3a_fused_residual_rmsnorm(dev):
    say("config 3a: fused residual + RMSNorm fp16 [2048, 4096]")
    r = tu.rng(3)
    res = tu.normal(r, (2048, 4096))
    dx = tu.normal(r, (2048, 4096))
    w = tu.normal(r, (4096,), 1.0, 0.05)
    ref_res, ref_y = oracle.residual_rmsnorm_rows(res, dx, w, EPS)
    res_d = to_dev(res)
    y = jinf_amd.residual_rmsnorm_rows(res_d, to_dev(dx), to_dev(w), EPS)
    assert tu.bits_equal(host(res_d), ref_res)
    worst = tu.assert_f16_close(host(y), ref_y, 2, "fused y")
    say(f"max ulp {worst}")


def test_fixture_fused_fp16(dev):
    say("committed fused residual+RMSNorm fixture")
    g = np.load(os.path.join(HERE, "golden", "kernels.npz"))
    res_d = to_dev(g["frn_res"])
    y = jinf_amd.residual_rmsnorm_rows(res_d, to_dev(g["frn_x"]), to_dev(g["frn_w"]), EPS)
    assert tu.bits_equal(host(res_d), g["frn_res_out"])
    tu.assert_f16_close(host(y), g["frn_y"], 2, "fixture y")


# Few rows (< 1024) of more than 128 chunks take the two-chunks-per-lane form:
# 8200 and 4104 leave the last lanes' second chunk (or both) past the row,
# 16384 fp16 is its widest row (1024 lanes), 1032 its narrowest (128 lanes).
@pytest.mark.parametrize("rows,n", [(64, 8192), (1, 4096), (7, 4104), (300, 512),
                                    (64, 8200), (3, 16384), (2, 1032)])
@pytest.mark.parametrize("act,wdt", [(np.float16, np.float16), (np.float16, np.float32),
                                     (np.float32, np.float32), (np.float32, np.float16)])
def test_rows_plain_and_fused(dev, rows, n, act, wdt):
    say(f"rows={rows} n={n} act={np.dtype(act).name} w={np.dtype(wdt).name}")
    r = tu.rng(rows * 7 + n)
    x = tu.normal(r, (rows, n), dtype=act)
    res = tu.normal(r, (rows, n), dtype=act)
    w = tu.normal(r, (n,), 1.0, 0.05, wdt)
    ref = oracle.rmsnorm_rows(x, w, EPS)
    got = host(jinf_amd.rmsnorm_rows(to_dev(x), to_dev(w), EPS))
    ref_res, ref_y = oracle.residual_rmsnorm_rows(res, x, w, EPS)
    res_d = to_dev(res)
    got_y = host(jinf_amd.residual_rmsnorm_rows(res_d, to_dev(x), to_dev(w), EPS))
    assert tu.bits_equal(host(res_d), ref_res)
    if act == np.float16:
        tu.assert_f16_close(got, ref, 2, "plain")
        tu.assert_f16_close(got_y, ref_y, 2, "fused")
    else:
        tu.assert_f32_close(got, ref, 1e-5, 1e-30, "plain")
        tu.assert_f32_close(got_y, ref_y, 1e-5, 1e-30, "fused")


def test_strided_rows_take_the_loop_path(dev):
    say("row stride 4100 fp16 (rows not 16-byte aligned)")
    r = tu.rng(12)
    big = tu.normal(r, (16, 4100))
    w = tu.normal(r, (4096,), 1.0, 0.05)
    x = to_dev(big)[:, 1:4097]
    out = torch.zeros((16, 4100), dtype=torch.float16, device=dev)
    jinf_amd.rmsnorm_rows(x, to_dev(w), EPS, out=out[:, 3:4099])
    o = host(out)
    ref = oracle.rmsnorm_rows(np.ascontiguousarray(big[:, 1:4097]), w, EPS)
    tu.assert_f16_close(o[:, 3:4099], ref, 2, "strided")
    assert np.all(o[:, :3] == 0) and np.all(o[:, 4099:] == 0)


def test_full_size_properties(dev):
    say("config 3a full size: scale invariance and unit RMS with w = 1")
    r = tu.rng(13)
    x = torch.from_numpy(tu.normal(r, (2048, 4096), dtype=np.float32)).to(dev)
    ones = torch.ones(4096, dtype=torch.float32, device=dev)
    y1 = jinf_amd.rmsnorm_rows(x, ones, 0.0)
    y2 = jinf_amd.rmsnorm_rows(x * 4.0, ones, 0.0)
    y1h, y2h = host(y1), host(y2)
    tu.assert_f32_close(y2h, y1h, 1e-6, 1e-30, "scale invariance")
    ms = np.mean(y1h.astype(np.float64) ** 2, axis=1)
    assert np.max(np.abs(ms - 1.0)) < 1e-5


def test_unsupported_weight_type_uses_fp32_like_reference(dev):
    say("drop-in weight_type 2 is read as fp32 (cuda/rmsnorm_kernel.cu:79-83)")
    r = tu.rng(14)
    x = tu.normal(r, (1, 512), 0.0, 1.0, np.float32)
    w = tu.normal(r, (512,), 1.0, 0.05, np.float32)
    out = torch.empty(512, dtype=torch.float32, device=dev)
    wd, xd = to_dev(w), to_dev(x[0])
    jinf_amd.lib().jinf_cuda_rmsnorm(ctypes.c_void_p(out.data_ptr()),
                                     ctypes.c_void_p(xd.data_ptr()),
                                     ctypes.c_void_p(wd.data_ptr()), 512, EPS, 2,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    tu.assert_f32_close(host(out), oracle.rmsnorm_rows(x, w, EPS)[0], 1e-5)
