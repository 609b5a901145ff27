"""The no-allocation entry point jinf_attention_decode_noalloc, through the
C-ABI, against jinf_attention_decode with a caller workspace.

Both run the same kernels with the same chunking, so the outputs must be
bit-identical (integer-exact bar: same arithmetic in the same order).  Each
case makes two calls in a row into the shared per-device scratch, the second
with a smaller input, so the second call runs on the first call's leftover
records and counters.  The cases cover the in-launch merge (few sequence /
head-group pairs), the separate merge launch (many pairs), unsplit contexts
(no scratch use), a shape whose split would need more records than the
scratch holds (it runs unsplit: the workspace entry point's bits without a
workspace), and the call captured in a HIP graph and replayed three times,
with eager work between the replays, each replay against the workspace entry
point's bits.
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


def _noalloc(out, q, k, v, lens, n_heads, n_kv):
    """jinf_attention_decode_noalloc over caches [n_seq, max_ctx, n_kv*hd]."""
    fn = jinf_amd.lib().jinf_attention_decode_noalloc
    n_seq, max_ctx, kvw = k.shape
    kv_type = jinf_amd.F16 if k.dtype == torch.float16 else jinf_amd.F32
    return fn(out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), k.data_ptr(),
              v.data_ptr(), kv_type, k.stride(1), k.stride(0), lens.data_ptr(), n_seq, max_ctx,
              kvw // n_kv, n_heads, n_kv, 0.0, torch.cuda.current_stream().cuda_stream)


def _case(r, n_seq, max_ctx, nh, nkv, hd, dtype=np.float16):
    lens = r.integers(1, max_ctx + 1, size=n_seq).astype(np.int32)
    lens[0] = max_ctx
    k = tu.normal(r, (n_seq, max_ctx, nkv * hd), 0.0, 1.0, np.float32).astype(dtype)
    v = tu.normal(r, (n_seq, max_ctx, nkv * hd), 0.0, 1.0, np.float32).astype(dtype)
    q = tu.normal(r, (n_seq, nh * hd), 0.0, 2.0, np.float32)
    return to_dev(q), to_dev(k), to_dev(v), to_dev(lens)


# (first call, second smaller call): (n_seq, max_ctx, n_heads, n_heads_kv, head_dim)
PAIRS = [
    # in-launch merge (4 pairs), then fewer positions
    ((1, 8192, 32, 8, 128), (1, 3000, 32, 8, 128)),
    # separate merge launch (512 pairs, the 70B decode shape), then 16 sequences
    ((64, 2048, 64, 8, 128), (16, 1024, 64, 8, 128)),
    # in-launch merge with head_dim 64, then a context within one chunk
    ((5, 2500, 16, 2, 64), (2, 200, 16, 2, 64)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_workspace_entry_point(dev, first, second):
    r = tu.rng(sum(first) + sum(second))
    for i, (n_seq, max_ctx, nh, nkv, hd) in enumerate((first, second)):
        say(f"call {i + 1}: n_seq={n_seq} ctx={max_ctx} heads={nh}/{nkv} hd={hd}")
        qd, kd, vd, ld = _case(r, n_seq, max_ctx, nh, nkv, hd)
        ws = jinf_amd.attention_workspace(n_seq, nh, hd, max_ctx)
        want = host(jinf_amd.attention_decode(qd, kd, vd, ld, nh, nkv, workspace=ws))
        out = torch.full((n_seq, nh * hd), float("nan"), dtype=torch.float32, device=dev)
        assert _noalloc(out, qd, kd, vd, ld, nh, nkv) == jinf_amd._lib.JINF_HIP_OK
        got = host(out)
        assert tu.bits_equal(got, want), f"call {i + 1}"
        if i == 1 and n_seq == 2:  # one small case also against the fp64 oracle
            oracle.set_threads(8)
            ref, a = oracle.attention(host(qd), host(kd), host(vd), host(ld), nh, nkv, hd)
            oracle.set_threads(1)
            err = np.abs(got.astype(np.float64) - ref) / np.maximum(a, 1e-30)
            assert float(err.max()) <= 2e-5


def test_noalloc_fp32_cache_needs_no_scratch(dev):
    say("fp32 cache (no split), 3 sequences x 700 positions")
    r = tu.rng(77)
    qd, kd, vd, ld = _case(r, 3, 700, 32, 8, 128, np.float32)
    want = host(jinf_amd.attention_decode(qd, kd, vd, ld, 32, 8))
    out = torch.empty((3, 32 * 128), dtype=torch.float32, device=dev)
    assert _noalloc(out, qd, kd, vd, ld, 32, 8) == jinf_amd._lib.JINF_HIP_OK
    assert tu.bits_equal(host(out), want)


def test_noalloc_runs_unsplit_beyond_the_scratch(dev):
    # 127 sequences x 8 head groups = 1016 pairs over 8192 positions: chunks
    # of 8128 positions (8192 * 1016 / 1024 items), so two per sequence, and
    # 127 * 64 * 2 * 130 * 4 = 8,453,120 bytes of records > 8 MiB
    # (8,388,608): the call runs unsplit, as the workspace entry point does
    # without a workspace, and gives its bits.
    say("127 x 8192 x 64/8 x 128: split would need more than the scratch; unsplit")
    n_seq, max_ctx, nh, nkv, hd = 127, 8192, 64, 8, 128
    g = torch.Generator(device=dev)
    g.manual_seed(127)
    k = torch.randn((n_seq, max_ctx, nkv * hd), generator=g, device=dev, dtype=torch.float16)
    v = torch.randn((n_seq, max_ctx, nkv * hd), generator=g, device=dev, dtype=torch.float16)
    q = torch.randn((n_seq, nh * hd), generator=g, device=dev) * 2.0
    lens = torch.randint(1, max_ctx + 1, (n_seq,), generator=g, device=dev, dtype=torch.int32)
    lens[0] = max_ctx
    want = host(jinf_amd.attention_decode(q, k, v, lens, nh, nkv))
    out = torch.full((n_seq, nh * hd), float("nan"), dtype=torch.float32, device=dev)
    assert _noalloc(out, q, k, v, lens, nh, nkv) == jinf_amd._lib.JINF_HIP_OK
    assert tu.bits_equal(host(out), want)


@pytest.mark.parametrize("shape", [(1, 8192, 32, 8, 128), (64, 2048, 64, 8, 128)])
def test_noalloc_captured_in_a_graph(dev, shape):
    """The in-launch merge (1 x 8192) and the separate merge launch (64 x
    2048) captured in a HIP graph after one lookup call (n_seq 0), replayed
    three times with eager work in between: every replay gives the workspace
    entry point's bits."""
    n_seq, max_ctx, nh, nkv, hd = shape
    say(f"graph capture: n_seq={n_seq} ctx={max_ctx} heads={nh}/{nkv} hd={hd}")
    r = tu.rng(sum(shape))
    qd, kd, vd, ld = _case(r, n_seq, max_ctx, nh, nkv, hd)
    ws = jinf_amd.attention_workspace(n_seq, nh, hd, max_ctx)
    want = host(jinf_amd.attention_decode(qd, kd, vd, ld, nh, nkv, workspace=ws))
    fn = jinf_amd.lib().jinf_attention_decode_noalloc
    # the lookup call: no sequences, nothing enqueued
    assert fn(0, 0, 0, 0, 0, 0, jinf_amd.F16, 0, 0, 0, 0, 0, hd, nh, nkv, 0.0,
              torch.cuda.current_stream().cuda_stream) == jinf_amd._lib.JINF_HIP_OK
    out = torch.full((n_seq, nh * hd), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _noalloc(out, qd, kd, vd, ld, nh, nkv)
    assert rc == jinf_amd._lib.JINF_HIP_OK
    for i in range(3):
        out.fill_(float("nan"))
        # eager work between replays, through the same scratch: a smaller call
        small = torch.empty((1, nh * hd), dtype=torch.float32, device=dev)
        assert _noalloc(small, qd[:1], kd[:1], vd[:1], ld[:1], nh, nkv) == jinf_amd._lib.JINF_HIP_OK
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert tu.bits_equal(host(out), want), f"replay {i + 1}"
