"""GPU parity: the fused layer GEMVs (include/jinf/kernels_ext.h:
jinf_rmsnorm_matvec, jinf_matvec_add, jinf_rmsnorm_swiglu_matvec,
jinf_rmsnorm_qkv_rope) against the oracle's composition of the unfused
reference launches they replace (RMSNorm, then the GEMV; the GEMV, then the
residual add; gate and up GEMVs, then SiLU * up; Q/K/V GEMVs, then RoPE and
the cache stores).

Bars (a = sum_j |w_j x_j| of a row, the dot product's own rounding scale):
- a GEMV output: |y - y_oracle| <= 1e-5 * a (as the plain GEMV's tests);
- + residual: 1e-5 * a + one fp32 rounding of the sum;
- SiLU(g) * u: the GEMV bars carried through the product,
  1e-5 * (1.1 |u| a_g + |silu(g)| a_u), plus 4 fp32 ulps of the result for
  SiLU's own exp and divide (|d silu/dg| <= 1.1);
- a RoPE pair: 1e-5 * (a_0 + a_1) on both rotated values, plus one fp16
  rounding step where the cache is fp16 (both sides round to fp16, and a
  value within the GEMV's error of a midpoint may round the other way).
"""
import numpy as np
import pytest
import torch

import jinf_amd
import oracle
import testutil as tu
from gpu_util import dev as to_dev
from gpu_util import host, say

pytestmark = pytest.mark.gpu

QTYPES = [oracle.Q4_0, oracle.Q8_0, oracle.Q4_K, oracle.Q6_K]
NAMES = {oracle.Q4_0: "Q4_0", oracle.Q8_0: "Q8_0", oracle.Q4_K: "Q4_K", oracle.Q6_K: "Q6_K"}
EPS = 1e-5


def mv(qtype, W, x):
    oracle.set_threads(8)
    try:
        return oracle.matvec(qtype, W, x)
    finally:
        oracle.set_threads(1)


def norm(h, g):
    return oracle.rmsnorm_rows(h[None], g, EPS)[0]


def check(got, ref, bound, what):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = float(np.max(err / np.maximum(bound, 1e-30)))
    say(f"{what}: worst error / bound = {worst:.2e}")
    assert np.all(np.isfinite(got)), what
    assert worst <= 1.0, what


def inputs(seed, qtype, rows, cols, g_dtype=np.float32):
    r = tu.rng(seed)
    W = tu.quant_table(r, qtype, rows, cols)
    h = tu.normal(r, (cols,), 0.0, 3.0, np.float32)
    g = tu.normal(r, (cols,), 1.0, 0.1, g_dtype)
    return r, W, h, g


# (rows, cols): Llama-3-8B q/o, k/v and output-sized slices, the 70B width
# (two tiles), and widths / offsets that take the generic kernel
SHAPES = [(4096, 4096), (1024, 4096), (3000, 8192)]


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("g_dtype", [np.float32, np.float16], ids=["g32", "g16"])
def test_rmsnorm_matvec(dev, qtype, rows, cols, g_dtype):
    say(f"rmsnorm_matvec {NAMES[qtype]} {rows}x{cols} g {g_dtype.__name__}")
    _, W, h, g = inputs(rows + cols + qtype, qtype, rows, cols, g_dtype)
    ref, a = mv(qtype, W, norm(h, g))
    y = host(jinf_amd.rmsnorm_matvec(to_dev(W), to_dev(h), qtype, to_dev(g), EPS))
    check(y, ref, 1e-5 * a, f"{NAMES[qtype]} {rows}x{cols}")


@pytest.mark.parametrize("qtype,rows,cols,h_off", [
    (oracle.Q4_0, 33, 384, 0), (oracle.Q8_0, 50, 160, 0), (oracle.Q4_0, 40, 4096, 1),
    (oracle.Q4_K, 21, 768, 0), (oracle.Q6_K, 9, 1280, 0), (oracle.Q6_K, 16, 4096, 3)])
def test_rmsnorm_matvec_generic(dev, qtype, rows, cols, h_off):
    say(f"rmsnorm_matvec generic {NAMES[qtype]} {rows}x{cols} h offset {h_off}")
    _, W, h, g = inputs(rows * 3 + cols, qtype, rows, cols)
    ref, a = mv(qtype, W, norm(h, g))
    hb = torch.zeros(cols + 4, dtype=torch.float32, device=dev)
    hb[h_off:h_off + cols] = to_dev(h)
    y = host(jinf_amd.rmsnorm_matvec(to_dev(W), hb[h_off:h_off + cols], qtype, to_dev(g), EPS))
    check(y, ref, 1e-5 * a, "generic")


def test_rmsnorm_matvec_without_norm_is_plain_matvec(dev):
    _, W, h, _ = inputs(5, oracle.Q4_0, 4096, 4096)
    Wd, hd = to_dev(W), to_dev(h)
    y0 = host(jinf_amd.matvec(Wd, hd, oracle.Q4_0))
    y1 = host(jinf_amd.rmsnorm_matvec(Wd, hd, oracle.Q4_0))
    assert tu.bits_equal(y0, y1)


def test_fused_norm_matches_rmsnorm_then_matvec(dev):
    """Same rs, same x^: the fused launch equals jinf_rmsnorm_rows followed by
    jinf_matvec bit for bit (both take the fp64 sum of squares)."""
    _, W, h, g = inputs(6, oracle.Q4_K, 4096, 4096)
    Wd, hd, gd = to_dev(W), to_dev(h), to_dev(g)
    xhat = jinf_amd.rmsnorm_rows(hd[None], gd, EPS)[0]
    y0 = host(jinf_amd.matvec(Wd, xhat, oracle.Q4_K))
    y1 = host(jinf_amd.rmsnorm_matvec(Wd, hd, oracle.Q4_K, gd, EPS))
    assert tu.bits_equal(y0, y1)


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (4096, 14336), (128, 384)])
def test_matvec_add(dev, qtype, rows, cols):
    if qtype in (oracle.Q4_K, oracle.Q6_K) and cols % 256:
        pytest.skip("width not whole K-format blocks")
    say(f"matvec_add {NAMES[qtype]} {rows}x{cols}")
    r, W, x, _ = inputs(rows + 7 * cols + qtype, qtype, rows, cols)
    y0 = tu.normal(r, (rows,), 0.0, 50.0, np.float32)
    ref, a = mv(qtype, W, x)
    yd = to_dev(y0)
    jinf_amd.matvec_add(to_dev(W), to_dev(x), qtype, yd)
    want = y0.astype(np.float64) + ref.astype(np.float64)
    check(host(yd), want, 1e-5 * a + np.abs(want) * 2.0 ** -24, f"{NAMES[qtype]} {rows}x{cols}")


def silu64(g):
    g = g.astype(np.float64)
    with np.errstate(over="ignore"):  # exp(-g) = inf for g < -709: silu = -0
        return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("n_ff,cols", [(14336, 4096), (1000, 8192), (96, 384)])
def test_rmsnorm_swiglu_matvec(dev, qtype, n_ff, cols):
    if qtype in (oracle.Q4_K, oracle.Q6_K) and cols % 256:
        pytest.skip("width not whole K-format blocks")
    say(f"rmsnorm_swiglu_matvec {NAMES[qtype]} n_ff={n_ff} cols={cols}")
    r, Wg, h, g = inputs(n_ff + cols + qtype, qtype, n_ff, cols)
    Wu = tu.quant_table(r, qtype, n_ff, cols)
    xh = norm(h, g)
    gr, ag = mv(qtype, Wg, xh)
    ur, au = mv(qtype, Wu, xh)
    want = silu64(gr) * ur.astype(np.float64)
    out = host(jinf_amd.rmsnorm_swiglu_matvec(to_dev(Wg), to_dev(Wu), to_dev(h), qtype,
                                              to_dev(g), EPS))
    bound = (1e-5 * (1.1 * np.abs(ur) * ag + np.abs(silu64(gr)) * au)
             + 4 * np.abs(want) * 2.0 ** -24)
    check(out, want, bound, f"{NAMES[qtype]} {n_ff}x{cols}")


def test_swiglu_fusion_equals_separate_launches(dev):
    """Gate and up GEMVs, then jinf_swiglu_rows, give the fused launch's bits."""
    r, Wg, h, g = inputs(9, oracle.Q4_0, 14336, 4096)
    Wu = tu.quant_table(r, oracle.Q4_0, 14336, 4096)
    Wgd, Wud, hd, gd = to_dev(Wg), to_dev(Wu), to_dev(h), to_dev(g)
    gt = jinf_amd.rmsnorm_matvec(Wgd, hd, oracle.Q4_0, gd, EPS)
    up = jinf_amd.rmsnorm_matvec(Wud, hd, oracle.Q4_0, gd, EPS)
    sep = host(jinf_amd.swiglu(gt, up))
    fused = host(jinf_amd.rmsnorm_swiglu_matvec(Wgd, Wud, hd, oracle.Q4_0, gd, EPS))
    assert tu.bits_equal(sep, fused)


def rope_ref(qv, kv, hd, pos, base):
    q2, k2 = oracle.rope_rows(qv[None], kv[None], hd, positions=[pos], base=base)
    return q2[0], k2[0]


def pair_bound(a):
    """1e-5 * (a_2i + a_2i+1) for both values of each pair."""
    s = a.reshape(-1, 2).sum(axis=1)
    return np.repeat(s, 2) * 1e-5


# (qtype, n_embd, n_heads, n_heads_kv, head_dim, kv dtype)
QKV = [(oracle.Q4_0, 4096, 32, 8, 128, np.float16), (oracle.Q4_K, 4096, 32, 8, 128, np.float32),
       (oracle.Q8_0, 4096, 32, 8, 128, np.float16), (oracle.Q6_K, 4096, 32, 8, 128, np.float16),
       (oracle.Q4_0, 8192, 64, 8, 128, np.float16), (oracle.Q4_0, 384, 4, 2, 96, np.float32),
       (oracle.Q8_0, 256, 4, 1, 64, np.float16)]


@pytest.mark.parametrize("qtype,n,nh,nkv,hd,kvdt", QKV)
def test_rmsnorm_qkv_rope(dev, qtype, n, nh, nkv, hd, kvdt):
    say(f"rmsnorm_qkv_rope {NAMES[qtype]} n={n} heads {nh}/{nkv}x{hd} cache {kvdt.__name__}")
    base, pos, max_ctx = 500000.0, 1234, 1500
    r, Wq, h, g = inputs(n + nh + hd + qtype, qtype, nh * hd, n)
    Wk = tu.quant_table(r, qtype, nkv * hd, n)
    Wv = tu.quant_table(r, qtype, nkv * hd, n)
    xh = norm(h, g)
    (qr, aq), (kr, ak), (vr, av) = mv(qtype, Wq, xh), mv(qtype, Wk, xh), mv(qtype, Wv, xh)
    q_want, k_want = rope_ref(qr, kr, hd, pos, base)
    tdt = torch.float16 if kvdt == np.float16 else torch.float32
    kc = torch.full((max_ctx, nkv * hd), -7.0, dtype=tdt, device=dev)
    vc = torch.full((max_ctx, nkv * hd), -7.0, dtype=tdt, device=dev)
    p = torch.tensor([pos], dtype=torch.int32, device=dev)
    q = host(jinf_amd.rmsnorm_qkv_rope(to_dev(Wq), to_dev(Wk), to_dev(Wv), to_dev(h), qtype, p,
                                       kc, vc, hd, nh, nkv, base, to_dev(g), EPS))
    check(q, q_want, pair_bound(aq) + np.abs(q_want) * 2.0 ** -23, "q")
    kh, vh = host(kc).astype(np.float32), host(vc).astype(np.float32)
    step = 2.0 ** -10 if kvdt == np.float16 else 2.0 ** -23
    check(kh[pos], k_want, pair_bound(ak) + np.abs(k_want) * step, "K row")
    check(vh[pos], vr, 1e-5 * av + np.abs(vr) * step, "V row")
    others = np.delete(np.arange(max_ctx), pos)
    assert np.all(kh[others] == -7.0) and np.all(vh[others] == -7.0)


def test_qkv_segments_and_position_outside_cache(dev):
    """Any subset of the three projections; a position past the cache keeps
    the cache untouched while q is still rotated at that position."""
    qtype, n, nh, nkv, hd = oracle.Q4_0, 4096, 32, 8, 128
    r, Wq, h, g = inputs(77, qtype, nh * hd, n)
    Wk = tu.quant_table(r, qtype, nkv * hd, n)
    Wv = tu.quant_table(r, qtype, nkv * hd, n)
    Wqd, Wkd, Wvd, hd_, gd = to_dev(Wq), to_dev(Wk), to_dev(Wv), to_dev(h), to_dev(g)
    kc = torch.zeros((64, nkv * hd), dtype=torch.float16, device=dev)
    vc = torch.zeros((64, nkv * hd), dtype=torch.float16, device=dev)
    p = torch.tensor([5], dtype=torch.int32, device=dev)
    full_q = host(jinf_amd.rmsnorm_qkv_rope(Wqd, Wkd, Wvd, hd_, qtype, p, kc, vc, hd, nh, nkv,
                                            1e4, gd, EPS))
    k_full, v_full = host(kc).copy(), host(vc).copy()
    kc.zero_()
    vc.zero_()
    # v alone, then q and k together: same bits
    assert jinf_amd.rmsnorm_qkv_rope(None, None, Wvd, hd_, qtype, p, kc, vc, hd, nh, nkv, 1e4,
                                     gd, EPS) is None
    q2 = host(jinf_amd.rmsnorm_qkv_rope(Wqd, Wkd, None, hd_, qtype, p, kc, vc, hd, nh, nkv, 1e4,
                                        gd, EPS))
    assert tu.bits_equal(q2, full_q)
    assert tu.bits_equal(host(kc), k_full) and tu.bits_equal(host(vc), v_full)
    # position 64 (= max_ctx): no cache store
    kc.zero_()
    vc.zero_()
    p64 = torch.tensor([64], dtype=torch.int32, device=dev)
    q3 = host(jinf_amd.rmsnorm_qkv_rope(Wqd, Wkd, Wvd, hd_, qtype, p64, kc, vc, hd, nh, nkv, 1e4,
                                        gd, EPS))
    assert np.all(host(kc) == 0) and np.all(host(vc) == 0)
    qr, aq = mv(qtype, Wq, norm(h, g))
    kr, _ = mv(qtype, Wk, norm(h, g))
    q_want, _ = rope_ref(qr, kr, hd, 64, 1e4)
    check(q3, q_want, pair_bound(aq) + np.abs(q_want) * 2.0 ** -23, "q at 64")
