"""Shared helpers for the jinf tests: seeded inputs and comparison metrics.

Inputs are drawn with numpy's PCG64 (np.random.default_rng(seed)) in float64
and rounded once to the storage type (numpy's float16 cast is RNE).  N(mu, s)
uses s as the standard deviation.
"""
import numpy as np

Q4_BLOCK = 18


def rng(seed):
    return np.random.default_rng(seed)


def normal(r, shape, mu=0.0, sigma=1.0, dtype=np.float16):
    return r.normal(mu, sigma, size=shape).astype(dtype)


def q4_0_table(r, n_rows, n_embd, scale_sigma=0.02):
    """Random Q4_0 table: d = fp16(|N(0, scale_sigma)|), nibbles uniform 0..15."""
    nb = n_embd // 32
    d = np.abs(r.normal(0.0, scale_sigma, size=(n_rows, nb))).astype(np.float16)
    qs = r.integers(0, 256, size=(n_rows, nb, 16), dtype=np.uint8)
    blk = np.empty((n_rows, nb, Q4_BLOCK), np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(n_rows, nb, 2)
    blk[:, :, 2:] = qs
    return blk.reshape(n_rows, nb * Q4_BLOCK)


def quant_table(r, qtype, n_rows, n_cols, scale_sigma=0.01):
    """Random weight rows of a GGUF block type (qtype codes 2, 8, 12, 14):
    binary16 scales fp16(|N(0, scale_sigma)|), every other byte uniform (Q6_K
    int8 sub-block scales included, so negative scales occur)."""
    if qtype == 2:
        return q4_0_table(r, n_rows, n_cols, scale_sigma)
    elems, nbytes = {8: (32, 34), 12: (256, 144), 14: (256, 210)}[qtype]
    nb = n_cols // elems
    blk = r.integers(0, 256, size=(n_rows, nb, nbytes), dtype=np.uint8)
    d = np.abs(r.normal(0.0, scale_sigma, size=(n_rows, nb))).astype(np.float16)
    dv = d.view(np.uint8).reshape(n_rows, nb, 2)
    if qtype == 8:
        blk[:, :, 0:2] = dv
    elif qtype == 12:
        blk[:, :, 0:2] = dv
        dmin = np.abs(r.normal(0.0, scale_sigma, size=(n_rows, nb))).astype(np.float16)
        blk[:, :, 2:4] = dmin.view(np.uint8).reshape(n_rows, nb, 2)
    else:
        blk[:, :, 208:210] = dv
    return blk.reshape(n_rows, nb * nbytes)


def extreme_quant_table(r, qtype, n_rows, n_cols):
    """quant_table rows whose codes and sub-block scales sit at their format's
    limits: Q4_0 nibbles 0 / 15; Q8_0 codes -128 / 127; Q4_K 6-bit scales and
    minimums all 63 (scale bytes 0xFF) with nibbles 0 / 15 (sc * q reaches
    945); Q6_K codes 0 / 63 (q - 32 = -32 / 31, high bits 00 / 11) under int8
    sub-block scales -128 / 127.  The fp16 block scales stay quant_table's."""
    W = quant_table(r, qtype, n_rows, n_cols).copy()
    elems, nbytes = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[qtype]
    B = W.reshape(n_rows, n_cols // elems, nbytes)

    def pick(choices, n):
        idx = r.integers(0, len(choices), size=B.shape[:2] + (n,))
        return np.asarray(choices, np.uint8)[idx]

    if qtype == 2:
        B[:, :, 2:18] = pick([0x00, 0xFF, 0x0F, 0xF0], 16)
    elif qtype == 8:
        B[:, :, 2:34] = pick([0x80, 0x7F], 32)
    elif qtype == 12:
        B[:, :, 4:16] = 0xFF
        B[:, :, 16:144] = pick([0x00, 0xFF, 0x0F, 0xF0], 128)
    else:
        B[:, :, 0:128] = pick([0x00, 0xFF, 0x0F, 0xF0], 128)
        B[:, :, 128:192] = pick([0x00, 0xFF, 0x33, 0xCC], 64)
        B[:, :, 192:208] = pick([0x80, 0x7F], 16)
    return B.reshape(n_rows, -1)


def q4_0_blocks(d_bits, qs):
    """Build blocks from fp16 scale bit patterns [n] and nibble bytes [n, 16]."""
    d_bits = np.asarray(d_bits, dtype=np.uint16)
    n = d_bits.shape[0]
    blk = np.empty((n, Q4_BLOCK), np.uint8)
    blk[:, 0:2] = d_bits.view(np.uint8).reshape(n, 2)
    blk[:, 2:] = np.asarray(qs, dtype=np.uint8).reshape(n, 16)
    return blk.reshape(-1)


def _ordinal16(a):
    b = np.asarray(a, dtype=np.float16).view(np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def ulp16(a, b):
    """fp16 ulp distance (0 between +0 and -0); NaN vs NaN is 0, NaN vs number huge."""
    a = np.asarray(a, dtype=np.float16)
    b = np.asarray(b, dtype=np.float16)
    d = np.abs(_ordinal16(a) - _ordinal16(b))
    na, nb = np.isnan(a), np.isnan(b)
    d = np.where(na & nb, 0, d)
    d = np.where(na ^ nb, 1 << 20, d)
    return d


def assert_f16_close(got, ref, max_ulp=2, what=""):
    d = ulp16(got, ref)
    worst = int(d.max()) if d.size else 0
    assert worst <= max_ulp, (
        f"{what}: max fp16 ulp distance {worst} > {max_ulp} "
        f"(first at {np.unravel_index(int(d.argmax()), d.shape)}: got "
        f"{np.asarray(got).reshape(-1)[int(d.argmax())]} ref {np.asarray(ref).reshape(-1)[int(d.argmax())]})")
    return worst


def rel_err_f32(got, ref, floor):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return np.abs(got - ref) / np.maximum(np.abs(ref), floor)


def assert_f32_close(got, ref, rel=1e-5, floor=1e-30, what=""):
    """|got - ref| <= rel * max(|ref|, floor)."""
    e = rel_err_f32(got, ref, floor)
    worst = float(e.max()) if e.size else 0.0
    assert worst <= rel, f"{what}: max relative error {worst:.3e} > {rel:.1e}"
    return worst


def bits_equal(a, b):
    """Bit-identical, with NaNs compared by class."""
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    ut = {2: np.uint16, 4: np.uint32}[a.dtype.itemsize]
    same = a.view(ut) == b.view(ut)
    same |= np.isnan(a) & np.isnan(b)
    return bool(same.all())
