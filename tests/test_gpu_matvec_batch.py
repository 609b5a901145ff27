"""GPU parity: the batched matrix-core GEMVs (include/jinf/kernels_ext.h:
jinf_matvec_batch, jinf_matvec_batch_add, jinf_rmsnorm_matvec_batch,
jinf_rmsnorm_swiglu_matvec_batch, jinf_rmsnorm_qkv_rope_batch) against the
oracle's per-token composition of the
reference launches (oracle.matvec on each sequence's vector, then the
residual add, SiLU * up, RoPE and the cache stores).

Bars, as for the one-token GEMVs (a = sum_j |w_j x_j| of a row, the dot
product's own rounding scale): a GEMV output |y - y_oracle| <= 1e-5 * a;
+ residual: 1e-5 * a + one fp32 rounding of the sum; SiLU(g) * u and RoPE
pairs carry the GEMV bars through as in test_gpu_fused.py.  The x halves
(fp16 hi + lo under a power-of-two scale per token) keep about 22 bits,
far inside these bars; rows of very different magnitudes in one batch, zero
rows and launches that split the columns exercise the scaling and the merge.
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


def mv_rows(qtype, W, X):
    ys, As = zip(*(mv(qtype, W, x) for x in X))
    return np.stack(ys), np.stack(As)


def check(got, ref, bound, what):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = float(np.max(err / np.maximum(bound, 1e-30)))
    say(f"{what}: worst error / bound = {worst:.2e}")
    assert np.all(np.isfinite(got)), what
    assert worst <= 1.0, what


def batch_x(r, n_batch, cols):
    """Rows of very different scales, one zero row when there is room."""
    X = tu.normal(r, (n_batch, cols), 0.0, 1.0, np.float32)
    scales = 10.0 ** np.linspace(-3, 4, n_batch)
    X *= scales[:, None].astype(np.float32)
    if n_batch > 2:
        X[1] = 0.0
    return X


# (rows, cols): 8B q/o, k/v, a ragged row count, a many-slab shape, an
# FFN-sized matrix and a ragged FFN-sized one (few column splits)
SHAPES = [(4096, 4096), (1024, 4096), (300, 2048), (64, 14336), (14336, 4096), (12300, 4096)]
BATCHES = [1, 13, 32, 64]


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("n_batch", BATCHES)
def test_matvec_batch(dev, qtype, rows, cols, n_batch):
    say(f"matvec_batch {NAMES[qtype]} {rows}x{cols} batch {n_batch}")
    r = tu.rng(rows + cols + 7 * qtype + n_batch)
    W = tu.quant_table(r, qtype, rows, cols)
    X = batch_x(r, n_batch, cols)
    ref, a = mv_rows(qtype, W, X)
    Wd, Xd = to_dev(W), to_dev(X)
    ws = jinf_amd.matvec_batch_workspace(rows, cols, n_batch)
    y = host(jinf_amd.matvec_batch(Wd, Xd, qtype, workspace=ws))
    check(y, ref, 1e-5 * a, "batch")
    # the workspace's counters are back at zero: a second call gives the same bits
    assert tu.bits_equal(host(jinf_amd.matvec_batch(Wd, Xd, qtype, workspace=ws)), y)
    if n_batch > 2:
        assert np.all(y[1] == 0.0)


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("rows,cols,n_batch", [(256, 4096, 32), (4096, 4096, 40),
                                               (64, 14336, 7)])
def test_matvec_batch_extreme_codes(dev, qtype, rows, cols, n_batch):
    """Every code and sub-block scale at its limit: the decodes into the
    matrix-core operands (one M-tile, two M-tiles, split columns) stay exact."""
    say(f"matvec_batch extreme codes {NAMES[qtype]} {rows}x{cols} batch {n_batch}")
    r = tu.rng(911 + qtype + rows + n_batch)
    W = tu.extreme_quant_table(r, qtype, rows, cols)
    X = batch_x(r, n_batch, cols)
    ref, a = mv_rows(qtype, W, X)
    ws = jinf_amd.matvec_batch_workspace(rows, cols, n_batch)
    y = host(jinf_amd.matvec_batch(to_dev(W), to_dev(X), qtype, workspace=ws))
    check(y, ref, 1e-5 * a, "extreme codes")


def test_matvec_batch_row_stride_and_one_token_agrees(dev):
    """Rows of x and y with padding between them; batch row b equals the
    batch-of-one result for x[b] up to the GEMV bar."""
    qtype, rows, cols = oracle.Q4_0, 512, 4096
    r = tu.rng(5)
    W = tu.quant_table(r, qtype, rows, cols)
    X = tu.normal(r, (5, cols), 0.0, 2.0, np.float32)
    Xpad = np.zeros((5, cols + 64), np.float32)
    Xpad[:, :cols] = X
    Wd = to_dev(W)
    Xd = to_dev(Xpad)[:, :cols]
    y = torch.full((5, rows + 8), -3.0, dtype=torch.float32, device=dev)
    jinf_amd.matvec_batch(Wd, Xd, qtype, y=y[:, :rows])
    yh = host(y)
    assert np.all(yh[:, rows:] == -3.0)
    ref, a = mv_rows(qtype, W, X)
    check(yh[:, :rows], ref, 1e-5 * a, "strided")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("n_batch", [3, 40])
def test_matvec_batch_add(dev, qtype, n_batch):
    rows, cols = 4096, 4096
    say(f"matvec_batch_add {NAMES[qtype]} batch {n_batch}")
    r = tu.rng(31 + qtype + n_batch)
    W = tu.quant_table(r, qtype, rows, cols)
    X = tu.normal(r, (n_batch, cols), 0.0, 1.0, np.float32)
    Y0 = tu.normal(r, (n_batch, rows), 0.0, 4.0, np.float32)
    ref, a = mv_rows(qtype, W, X)
    want = (Y0 + ref).astype(np.float32)
    yd = to_dev(Y0)
    jinf_amd.matvec_batch_add(to_dev(W), to_dev(X), qtype, yd)
    check(host(yd), want, 1e-5 * a + np.abs(want) * 2.0 ** -23, "y + W x")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
@pytest.mark.parametrize("g_dtype", [np.float32, np.float16], ids=["g32", "g16"])
def test_rmsnorm_matvec_batch(dev, qtype, g_dtype):
    rows, cols, n_batch = 2048, 4096, 24
    say(f"rmsnorm_matvec_batch {NAMES[qtype]} g {g_dtype.__name__}")
    r = tu.rng(61 + qtype)
    W = tu.quant_table(r, qtype, rows, cols)
    H = batch_x(r, n_batch, cols)
    H[1] = tu.normal(r, (cols,), 0.0, 1.0, np.float32)  # the norm needs a nonzero row
    g = tu.normal(r, (cols,), 1.0, 0.1, g_dtype)
    Xn = oracle.rmsnorm_rows(H, g, EPS)
    ref, a = mv_rows(qtype, W, Xn)
    Hd = to_dev(H)
    ws = jinf_amd.matvec_batch_workspace(rows, cols, n_batch)
    y = host(jinf_amd.rmsnorm_matvec_batch(to_dev(W), Hd, qtype, to_dev(g), EPS, workspace=ws))
    check(y, ref, 1e-5 * a, "rmsnorm + GEMV")
    # norm weights that are not 16-byte aligned (element loads): the same bits
    gbuf = to_dev(np.concatenate([np.zeros(1, g_dtype), g]))
    y1 = host(jinf_amd.rmsnorm_matvec_batch(to_dev(W), Hd, qtype, gbuf[1:], EPS, workspace=ws))
    assert np.array_equal(y1.view(np.uint32), y.view(np.uint32))
    # no norm weight: the plain batched GEMV of h
    ref2, a2 = mv_rows(qtype, W, H)
    y2 = host(jinf_amd.rmsnorm_matvec_batch(to_dev(W), Hd, qtype, None, EPS, workspace=ws))
    check(y2, ref2, 1e-5 * a2, "norm_w None")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: NAMES[q])
def test_rmsnorm_swiglu_matvec_batch(dev, qtype):
    n_ff, cols, n_batch = 14336, 4096, 9
    say(f"rmsnorm_swiglu_matvec_batch {NAMES[qtype]}")
    r = tu.rng(71 + qtype)
    Wg = tu.quant_table(r, qtype, n_ff, cols)
    Wu = tu.quant_table(r, qtype, n_ff, cols)
    H = tu.normal(r, (n_batch, cols), 0.0, 3.0, np.float32)
    g = tu.normal(r, (cols,), 1.0, 0.1, np.float32)
    Xn = oracle.rmsnorm_rows(H, g, EPS)
    gr, ag = mv_rows(qtype, Wg, Xn)
    ur, au = mv_rows(qtype, Wu, Xn)
    want = oracle.swiglu(gr, ur)
    Hd = to_dev(H)
    ws = jinf_amd.matvec_batch_workspace(n_ff, cols, n_batch)
    out = host(jinf_amd.rmsnorm_swiglu_matvec_batch(to_dev(Wg), to_dev(Wu), Hd, qtype,
                                                    to_dev(g), EPS, workspace=ws))
    sg = np.abs(want / np.where(ur == 0, 1, ur))
    bound = 1e-5 * (1.1 * np.abs(ur) * ag + sg * au) + np.abs(want) * 4 * 2.0 ** -23
    check(out, want, bound, "silu(gate) * up")


def rope_ref(qv, kv, hd, pos, base):
    q2, k2 = oracle.rope_rows(qv[None], kv[None], hd, positions=[pos], base=base)
    return q2[0], k2[0]


def pair_bound(a):
    s = a.reshape(-1, 2).sum(axis=1)
    return np.repeat(s, 2) * 1e-5


@pytest.mark.parametrize("qtype,n,nh,nkv,hd,kvdt", [
    (oracle.Q4_0, 4096, 32, 8, 128, np.float16), (oracle.Q4_K, 4096, 32, 8, 128, np.float32),
    (oracle.Q6_K, 4096, 32, 8, 128, np.float16), (oracle.Q8_0, 512, 8, 2, 64, np.float16)])
def test_rmsnorm_qkv_rope_batch(dev, qtype, n, nh, nkv, hd, kvdt):
    say(f"rmsnorm_qkv_rope_batch {NAMES[qtype]} n={n} heads {nh}/{nkv}x{hd}")
    base, max_ctx, n_batch = 500000.0, 300, 6
    positions = np.array([0, 17, 299, -1, 300, 5], np.int32)  # -1 and 300: no cache store
    r = tu.rng(n + nh + qtype)
    Wq = tu.quant_table(r, qtype, nh * hd, n)
    Wk = tu.quant_table(r, qtype, nkv * hd, n)
    Wv = tu.quant_table(r, qtype, nkv * hd, n)
    H = tu.normal(r, (n_batch, n), 0.0, 3.0, np.float32)
    g = tu.normal(r, (n,), 1.0, 0.1, np.float32)
    Xn = oracle.rmsnorm_rows(H, g, EPS)
    tdt = torch.float16 if kvdt == np.float16 else torch.float32
    kc = torch.full((n_batch, max_ctx, nkv * hd), -7.0, dtype=tdt, device=dev)
    vc = torch.full((n_batch, max_ctx, nkv * hd), -7.0, dtype=tdt, device=dev)
    Hd = to_dev(H)
    ws = jinf_amd.matvec_batch_workspace(nh * hd + 2 * nkv * hd, n, n_batch)
    q = host(jinf_amd.rmsnorm_qkv_rope_batch(
        to_dev(Wq), to_dev(Wk), to_dev(Wv), Hd, qtype, to_dev(g), to_dev(positions), kc, vc, hd,
        nh, nkv, base, EPS, workspace=ws))
    kh, vh = host(kc).astype(np.float32), host(vc).astype(np.float32)
    step = 2.0 ** -10 if kvdt == np.float16 else 2.0 ** -23
    for b in range(n_batch):
        (qr, aq), (kr, ak), (vr, av) = mv(qtype, Wq, Xn[b]), mv(qtype, Wk, Xn[b]), mv(qtype, Wv, Xn[b])
        pos = int(positions[b])
        q_want, k_want = rope_ref(qr, kr, hd, pos, base)
        check(q[b], q_want, pair_bound(aq) + np.abs(q_want) * 2.0 ** -23, f"q[{b}]")
        others = np.arange(max_ctx)
        if 0 <= pos < max_ctx:
            check(kh[b, pos], k_want, pair_bound(ak) + np.abs(k_want) * step, f"K[{b}]")
            check(vh[b, pos], vr, 1e-5 * av + np.abs(vr) * step, f"V[{b}]")
            others = np.delete(others, pos)
        assert np.all(kh[b, others] == -7.0) and np.all(vh[b, others] == -7.0)


def test_batch_rejections(dev):
    W = torch.zeros((64, 144), dtype=torch.uint8, device=dev)  # Q4_0 64 x 256
    x = torch.zeros((2, 256), dtype=torch.float32, device=dev)
    with pytest.raises(jinf_amd.JinfError):
        jinf_amd.matvec_batch(W, torch.zeros((65, 256), dtype=torch.float32, device=dev),
                              oracle.Q4_0)  # more than 64 sequences
    W2 = torch.zeros((64, 18 * 4), dtype=torch.uint8, device=dev)  # 128 columns
    with pytest.raises(jinf_amd.JinfError):
        jinf_amd.matvec_batch(W2, torch.zeros((2, 128), dtype=torch.float32, device=dev),
                              oracle.Q4_0)  # not whole 256-column slabs
    with pytest.raises(jinf_amd.JinfError):
        jinf_amd.matvec_batch(W, x[:, 1:], oracle.Q4_0)  # x not 16-byte aligned
    small = torch.zeros(256, dtype=torch.uint8, device=dev)
    with pytest.raises(jinf_amd.JinfError):
        jinf_amd.matvec_batch(W, x, oracle.Q4_0, workspace=small)  # workspace too small
