"""GPU: every jinf kernel captured into a HIP graph (torch.cuda.CUDAGraph on
torch's capture stream) gives, on every replay, exactly the bits of the eager
launch.  Replays are interleaved with eager work and synchronizations, and
in-place kernels get their inputs restored eagerly before each replay."""
import numpy as np
import pytest
import torch

import jinf_amd
import testutil as tu
from gpu_util import dev as to_dev
from gpu_util import host, say

pytestmark = pytest.mark.gpu


def _graph(fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_all_kernels_replay_bit_identical(dev):
    r = tu.rng(91)
    x = to_dev(tu.normal(r, (64, 4096)))
    res0 = to_dev(tu.normal(r, (64, 4096)))
    w = to_dev(tu.normal(r, (4096,), 1.0, 0.05))
    q0 = to_dev(tu.normal(r, (64, 32 * 128)))
    k0 = to_dev(tu.normal(r, (64, 8 * 128)))
    pos = to_dev(r.integers(0, 8192, size=64).astype(np.int32))
    gate = to_dev(tu.normal(r, (64, 14336), 0.0, 2.0))
    up = to_dev(tu.normal(r, (64, 14336), 0.0, 2.0))
    s = to_dev(tu.normal(r, (256, 8192), 0.0, 3.0, np.float32))
    lens = to_dev((r.integers(0, 8192, size=4) + 1).astype(np.int32))
    table = to_dev(tu.q4_0_table(r, 1000, 4096))
    ids = to_dev(r.integers(0, 1000, size=64).astype(np.int32))

    outs = {n: None for n in ("norm", "fres", "fy", "q", "k", "sw", "sm", "emb")}
    bufs = {
        "norm": torch.empty_like(x), "fres": torch.empty_like(res0), "fy": torch.empty_like(x),
        "q": torch.empty_like(q0), "k": torch.empty_like(k0), "sw": torch.empty_like(gate),
        "sm": torch.zeros_like(s), "emb": torch.empty((64, 4096), dtype=torch.float16, device=dev),
    }

    def reset():
        bufs["fres"].copy_(res0)
        bufs["q"].copy_(q0)
        bufs["k"].copy_(k0)
        bufs["sm"].zero_()

    def launch_all():
        jinf_amd.rmsnorm_rows(x, w, 1e-5, out=bufs["norm"])
        jinf_amd.residual_rmsnorm_rows(bufs["fres"], x, w, 1e-5, out=bufs["fy"])
        jinf_amd.rope_rows(bufs["q"], bufs["k"], 128, pos, 0, 500000.0)
        jinf_amd.swiglu(gate, up, out=bufs["sw"])
        jinf_amd.softmax_rows(s, lens, 64, 1.0, out=bufs["sm"])
        jinf_amd.embed_q4_0(table, ids, 4096, torch.float16, out=bufs["emb"])

    reset()
    launch_all()
    eager = {n: host(b).copy() for n, b in bufs.items()}
    reset()
    torch.cuda.synchronize()
    g = _graph(launch_all)
    for rep in range(4):
        say(f"replay {rep}")
        reset()
        _ = (x * 2).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n, b in bufs.items():
            assert tu.bits_equal(host(b), eager[n]), f"replay {rep}: {n}"


@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rmsnorm"])
def test_tall_gemv_replays_bit_identical(dev, norm):
    """The tall one-tile GEMV (rows >= 32768, Q6_K; its grid is the device's
    resident workgroup count, queried once per process, also under capture)
    captured in a graph: every replay, between eager launches of its own,
    gives the eager bits."""
    import oracle
    r = tu.rng(93 + norm)
    rows, cols = 40000, 4096
    W = to_dev(tu.quant_table(r, oracle.Q6_K, rows, cols))
    x = to_dev(tu.normal(r, (cols,), 0.0, 1.0, np.float32))
    g = to_dev(tu.normal(r, (cols,), 1.0, 0.1, np.float32))
    y = torch.empty(rows, dtype=torch.float32, device=dev)

    def run(out):
        if norm:
            jinf_amd.rmsnorm_matvec(W, x, oracle.Q6_K, norm_w=g, eps=1e-5, y=out)
        else:
            jinf_amd.matvec(W, x, oracle.Q6_K, y=out)

    # captured before any eager launch: in a process with no earlier tall
    # launch the grid query runs under the capture
    graph = _graph(lambda: run(y))
    want = torch.empty_like(y)
    run(want)
    for i in range(3):
        y.fill_(-1.0)
        graph.replay()
        torch.cuda.synchronize()
        say(f"tall gemv replay {i} ({'rmsnorm' if norm else 'plain'})")
        assert tu.bits_equal(host(y), host(want)), f"replay {i}"
        run(want)  # eager work between the replays
        torch.cuda.synchronize()
