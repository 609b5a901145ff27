"""GPU check of the bandwidth probes (include/jinf/probe_hip.h) behind every
kernel's ceiling and attainable rate in bench.py: each probe must move exactly
the bytes it claims, every launch layout and store order included, or the
ceilings it sets would be wrong.  A probe's stored unit is its loaded unit with
at most the lowest bit of the first word flipped; outputs start as a sentinel
(all ones), so a unit the probe skipped, or one written from the wrong input
unit, shows."""
import pytest
import torch

from gpu_util import say
from jinf_amd import ops

pytestmark = pytest.mark.gpu

SENTINEL = -1
LAYOUT_SHAPES = ((64, 0), (128, 0), (256, 0), (512, 0), (1024, 0), (256, 2048), (1024, 512), (64, 3))


def words(t):
    return t.view(torch.int32).reshape(-1, 4)


def assert_moved(out_words, in_words, what):
    assert torch.equal(out_words[:, 1:], in_words[:, 1:]), what
    assert int(((out_words[:, 0] ^ in_words[:, 0]) & ~1).abs().max()) == 0, what


def rand_words(n_units, g):
    return torch.randint(-2**31, 2**31 - 1, (n_units * 4,), generator=g, device="cuda",
                         dtype=torch.int32)


def test_stream_layouts_move_every_unit(dev):
    """jinf_probe_stream_layout, every layout and store order, 1 or 2 inputs and
    outputs, a unit count that leaves partial workgroups and stride loops."""
    g = torch.Generator(device="cuda").manual_seed(11)
    n = 5003
    in0, in1 = rand_words(n, g), rand_words(n, g)
    cases = 0
    for u in (1, 2, 4):
        for x in (False, True, 2):
            for b, gr in LAYOUT_SHAPES:
                for two_out in (True, False):
                    out0 = torch.full_like(in0, SENTINEL)
                    out1 = torch.full_like(in1, SENTINEL) if two_out else None
                    ops.probe_stream_layout(out0, in0, out1, in1, u, x, b, gr)
                    torch.cuda.synchronize()
                    what = f"units {u} order {x} lanes {b} groups {gr} outputs {1 + two_out}"
                    assert_moved(words(out0), words(in0), what)
                    if two_out:
                        assert_moved(words(out1), words(in1), what)
                    cases += 1
    say(f"{cases} stream layouts checked")


def test_stream_probe_in_place_and_one_input(dev):
    """jinf_probe_stream (the own-geometry flat probe) in place, and with one input."""
    g = torch.Generator(device="cuda").manual_seed(12)
    n = 3001
    for u in (1, 2, 4):
        for x in (True, False):
            a, b = rand_words(n, g), rand_words(n, g)
            a0, b0 = a.clone(), b.clone()
            ops.probe_stream(a, a, torch.full_like(b, SENTINEL), b, u, x)
            out = torch.full_like(a, SENTINEL)
            ops.probe_stream(out, b0, None, None, u, x)
            torch.cuda.synchronize()
            assert_moved(words(a), words(a0), f"in place, units {u} exchange {x}")
            assert_moved(words(out), words(b0), f"one input, units {u} exchange {x}")


def test_read_layouts_leave_sink(dev):
    g = torch.Generator(device="cuda").manual_seed(13)
    inp = rand_words(7001, g)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for u in (1, 2, 4):
        for b, gr in LAYOUT_SHAPES:
            ops.probe_read_layout(inp, sink, u, b, gr)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0


def test_rows_inplace_keeps_padding(dev):
    """RoPE's geometry: live units of both row sets moved, the padding past
    each row's live units untouched."""
    g = torch.Generator(device="cuda").manual_seed(14)
    T, na, nb, pad = 37, 70, 18, 6
    for u in (1, 2, 4):
        for x in (True, False):
            a = rand_words(T * (na + pad), g).reshape(T, (na + pad) * 4)
            b = rand_words(T * (nb + pad), g).reshape(T, (nb + pad) * 4)
            a0, b0 = a.clone(), b.clone()
            ops.probe_rows_inplace(a[:, :na * 4], b[:, :nb * 4], u, x)
            torch.cuda.synchronize()
            assert_moved(words(a), words(a0), f"a, units {u} exchange {x}")
            assert_moved(words(b), words(b0), f"b, units {u} exchange {x}")
            assert torch.equal(a[:, na * 4:], a0[:, na * 4:]) and torch.equal(b[:, nb * 4:], b0[:, nb * 4:])


def test_gather_rows_and_out_of_range_ids(dev):
    """Output unit v of row r comes from table unit floor(v * in / out) of row
    ids[r]; an id outside the table reads nothing (zeros, one bit at most)."""
    g = torch.Generator(device="cuda").manual_seed(15)
    rows, in_u, out_u = 300, 9, 32
    table = rand_words(rows * in_u, g).reshape(rows, in_u * 4)
    ids = torch.randint(0, rows, (41,), generator=g, device="cuda", dtype=torch.int32)
    ids[3], ids[17], ids[40] = -1, rows, 2**31 - 1
    src = torch.clamp((torch.arange(out_u) * in_u) // out_u, max=in_u - 1).to("cuda")
    for u in (1, 2, 4):
        for x in (True, False):
            out = torch.full((ids.numel(), out_u * 4), SENTINEL, dtype=torch.int32, device="cuda")
            ops.probe_gather(out, table.view(torch.uint8), ids, in_u * 16, u, x)
            torch.cuda.synchronize()
            ok = (ids >= 0) & (ids < rows)
            expect = torch.zeros((ids.numel(), out_u, 4), dtype=torch.int32, device="cuda")
            tw = table.reshape(rows, in_u, 4)
            expect[ok] = tw[ids[ok].long()][:, src]
            assert_moved(out.reshape(-1, 4), expect.reshape(-1, 4), f"units {u} exchange {x}")


def test_ragged_rows_move_live_units_only(dev):
    """The masked softmax's geometry: row r moves its first 4 floor(L / 4)
    floats (L = lens[r / rows_per_len] clamped to [0, n_cols]) and nothing past them."""
    g = torch.Generator(device="cuda").manual_seed(16)
    for n_cols in (200, 4096, 8192):
        rpl, groups = 3, 5
        R = rpl * groups
        x = torch.randn((R, n_cols), generator=g, device="cuda")
        lens = torch.tensor([0, 7, n_cols // 2 + 5, n_cols, n_cols + 9], dtype=torch.int32, device="cuda")
        out = torch.full((R, n_cols), float("nan"), device="cuda")
        ops.probe_rows_ragged(out, x, lens, rpl)
        torch.cuda.synchronize()
        for r in range(R):
            L = min(max(int(lens[r // rpl]), 0), n_cols) // 4 * 4
            ow, xw = out[r].view(torch.int32), x[r].view(torch.int32)
            if L:
                assert_moved(ow[:L].reshape(-1, 4), xw[:L].reshape(-1, 4), f"n_cols {n_cols} row {r}")
            assert torch.isnan(out[r, L:]).all(), f"n_cols {n_cols} row {r}: past its live units"
