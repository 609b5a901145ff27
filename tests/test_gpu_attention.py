"""GPU parity: GQA decode attention (jinf_cuda_attention / jinf_attention_decode)
against the oracle's fp64 attention.

Bar: |out - out_oracle| <= 2e-5 * sum_t p_t |v_t[d]| per output element (the
scale of the weighted sum's own rounding; the fp32 score carries a relative
error of a few ulp of sum |q k| / sqrt(hd), which moves each p_t by about as
much).  Cache positions at or past each length are filled with NaN, so a read
of the masked tail fails the test.
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


def check(out, ref, a, what, tol=2e-5):
    err = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    assert np.all(np.isfinite(out)), what
    worst = float(np.max(err / np.maximum(a, 1e-30)))
    say(f"{what}: worst error / sum p|v| = {worst:.2e}")
    assert worst <= tol, what


def make(r, n_seq, max_ctx, nh, nkv, hd, lens, dtype=np.float32, qsigma=1.0):
    k = tu.normal(r, (n_seq, max_ctx, nkv * hd), 0.0, 1.0, np.float32).astype(dtype)
    v = tu.normal(r, (n_seq, max_ctx, nkv * hd), 0.0, 1.0, np.float32).astype(dtype)
    q = tu.normal(r, (n_seq, nh * hd), 0.0, qsigma, np.float32)
    kp, vp = k.copy(), v.copy()
    for s, L in enumerate(lens):
        kp[s, max(L, 0):] = np.nan
        vp[s, max(L, 0):] = np.nan
    return q, k, v, kp, vp


def _oracle(q, k, v, lens, nh, nkv, hd, max_ctx):
    oracle.set_threads(8)
    try:
        return oracle.attention(q, k, v, np.clip(lens, 0, max_ctx), nh, nkv, hd)
    finally:
        oracle.set_threads(1)


@pytest.mark.parametrize("n_past", [1, 5, 64, 65, 1000, 4096])
def test_drop_in_llama_8b(dev, n_past):
    say(f"jinf_cuda_attention 32/8 heads x 128, n_past={n_past}, max_ctx=4096")
    nh, nkv, hd, max_ctx = 32, 8, 128, 4096
    r = tu.rng(n_past)
    q, k, v, kp, vp = make(r, 1, max_ctx, nh, nkv, hd, [n_past], qsigma=2.0)
    ref, a = _oracle(q, k, v, np.array([n_past]), nh, nkv, hd, max_ctx)
    out = torch.full((nh * hd,), -3.0, dtype=torch.float32, device=dev)
    jinf_amd.cuda_attention(out, to_dev(q[0]), to_dev(kp[0]), to_dev(vp[0]), hd, nh, nkv, n_past,
                            max_ctx)
    check(host(out)[None], ref, a, f"n_past={n_past}")


def test_drop_in_no_op_for_empty_context(dev):
    out = torch.full((256,), -3.0, dtype=torch.float32, device=dev)
    z = torch.zeros(4096, dtype=torch.float32, device=dev)
    jinf_amd.cuda_attention(out, z, z, z, 128, 2, 1, 0, 16)
    assert np.all(host(out) == -3.0)


# (n_seq, max_ctx, n_heads, n_heads_kv, head_dim, kv dtype): fp16 caches run
# the matrix-core kernel (GQA groups of 8, 4, 2 and 1 query heads per
# workgroup slot set, head_dim 64 and 128); fp32 caches the VALU kernel (one
# query head per workgroup for few (sequence, kv head) pairs, groups of 4
# otherwise); head_dim 96 and 80 the generic kernel.
CASES = [(8, 8192, 64, 8, 128, np.float16),   # 70B heads, long ragged contexts
         (16, 2048, 64, 8, 128, np.float16),  # G = 8
         (16, 1024, 32, 8, 128, np.float32),  # G = 4
         (32, 512, 8, 4, 128, np.float16),    # G = 2
         (64, 300, 16, 4, 64, np.float32),    # G = 4, head_dim 64
         (4, 700, 16, 2, 64, np.float16),     # one head per workgroup, head_dim 64
         (3, 200, 12, 4, 96, np.float32),     # generic kernel
         (2, 130, 6, 6, 80, np.float16)]      # generic kernel, MHA


@pytest.mark.parametrize("n_seq,max_ctx,nh,nkv,hd,dtype", CASES)
def test_batched_decode(dev, n_seq, max_ctx, nh, nkv, hd, dtype):
    say(f"jinf_attention_decode n_seq={n_seq} ctx={max_ctx} heads={nh}/{nkv} hd={hd} {dtype.__name__}")
    r = tu.rng(n_seq * 7 + hd + nh)
    lens = r.integers(1, max_ctx + 1, size=n_seq).astype(np.int32)
    lens[0] = 1
    lens[-1] = max_ctx
    q, k, v, kp, vp = make(r, n_seq, max_ctx, nh, nkv, hd, lens, dtype, qsigma=2.0)
    ref, a = _oracle(q, k, v, lens, nh, nkv, hd, max_ctx)
    out = host(jinf_amd.attention_decode(to_dev(q), to_dev(kp), to_dev(vp), to_dev(lens), nh, nkv))
    check(out, ref, a, f"{n_seq}x{nh}/{nkv}x{hd}")


def test_zero_and_overlong_lengths(dev):
    say("lens 0 -> zeros; lens > max_ctx -> clamped to max_ctx")
    n_seq, max_ctx, nh, nkv, hd = 3, 100, 8, 2, 128
    r = tu.rng(9)
    lens = np.array([0, 100000, 37], np.int32)
    q, k, v, _, _ = make(r, n_seq, max_ctx, nh, nkv, hd, [max_ctx] * 3)
    ref, a = _oracle(q, k, v, lens, nh, nkv, hd, max_ctx)
    out = host(jinf_amd.attention_decode(to_dev(q), to_dev(k), to_dev(v), to_dev(lens), nh, nkv))
    assert np.all(out[0] == 0.0)
    check(out[1:], ref[1:], a[1:], "clamped")


def test_explicit_scale_and_single_position(dev):
    say("scale argument; one position returns its value row exactly")
    n_seq, max_ctx, nh, nkv, hd = 2, 64, 8, 2, 128
    r = tu.rng(10)
    lens = np.array([1, 64], np.int32)
    q, k, v, kp, vp = make(r, n_seq, max_ctx, nh, nkv, hd, lens)
    out = host(jinf_amd.attention_decode(to_dev(q), to_dev(kp), to_dev(vp), to_dev(lens), nh, nkv,
                                         scale=0.5))
    for h in range(nh):
        assert tu.bits_equal(out[0, h * hd:(h + 1) * hd], v[0, 0, (h // 4) * hd:(h // 4 + 1) * hd])
    oracle.set_threads(8)
    ref, a = oracle.attention(q, k, v, lens, nh, nkv, hd, scale=0.5)
    oracle.set_threads(1)
    check(out, ref, a, "scale 0.5")


# Split of long contexts over workgroups through a workspace (fp16 caches):
# several chunks per sequence, a sequence shorter than one chunk, one that
# ends exactly on a chunk boundary, and batch 1.  Up to 127 (sequence, head
# group) pairs merge inside the attention launch; the last case (256 pairs)
# merges in a second launch.
SPLIT = [(8, 8192, 64, 8, 128), (3, 3000, 32, 8, 128), (1, 8192, 32, 8, 128),
         (5, 2500, 16, 2, 64), (32, 1024, 32, 8, 128)]


@pytest.mark.parametrize("n_seq,max_ctx,nh,nkv,hd", SPLIT)
def test_split_contexts_with_workspace(dev, n_seq, max_ctx, nh, nkv, hd):
    say(f"jinf_attention_decode + workspace n_seq={n_seq} ctx={max_ctx} heads={nh}/{nkv} hd={hd}")
    r = tu.rng(n_seq * 13 + max_ctx)
    lens = r.integers(1, max_ctx + 1, size=n_seq).astype(np.int32)
    lens[0] = max_ctx
    if n_seq > 2:
        lens[1] = 1000
        lens[2] = 2048
    q, k, v, kp, vp = make(r, n_seq, max_ctx, nh, nkv, hd, lens, np.float16, qsigma=2.0)
    ref, a = _oracle(q, k, v, lens, nh, nkv, hd, max_ctx)
    ws = jinf_amd.attention_workspace(n_seq, nh, hd, max_ctx)
    counters = (n_seq * nh * 4 + 255) // 256 * 256
    assert ws.numel() == counters + n_seq * nh * ((max_ctx + 255) // 256) * (hd + 2) * 4
    qd, kd, vd, ld = to_dev(q), to_dev(kp), to_dev(vp), to_dev(lens)
    out = host(jinf_amd.attention_decode(qd, kd, vd, ld, nh, nkv, workspace=ws))
    check(out, ref, a, f"split {n_seq}x{nh}/{nkv}x{hd}")
    # the merge counters are back at zero, and a second call with the same
    # workspace gives the same bits
    assert np.all(host(ws[:counters]) == 0)
    again = host(jinf_amd.attention_decode(qd, kd, vd, ld, nh, nkv, workspace=ws))
    assert tu.bits_equal(again, out)
    # the same call without a workspace (one work item per sequence)
    out1 = host(jinf_amd.attention_decode(qd, kd, vd, ld, nh, nkv))
    check(out1, ref, a, "unsplit")
