"""GPU parity: Q4_0 token-embedding gather / dequant, bit-exact.

Checked against the reference's own CPU dequantizer output (golden fixture
written from src/quant.cpp compiled in place) and against the oracle
(src/quant.cpp:49-60 semantics, engine row addressing src/engine.cpp:311-317)
at the full config-4 size, at the 70B row width, with out-of-range ids, and
on every staging-width / store-width path the launcher can pick.
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


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_reference_fixture_via_drop_in(dev):
    say("drop-in jinf_cuda_dequantize_q4_0 on the reference fixture (special scales, every byte)")
    g = np.load(os.path.join(HERE, "golden", "q4_0_ref.npz"))
    blocks, expect = g["blocks"], g["out"]
    nb = blocks.size // 18
    out = torch.full((nb * 32,), float("nan"), dtype=torch.float32, device=dev)
    jinf_amd.cuda_dequantize_q4_0(to_dev(blocks), out, nb)
    assert tu.bits_equal(host(out), expect)


def test_reference_fixture_fp16_gather(dev):
    say("fixture blocks as a 31-row table, fp16 gather")
    g = np.load(os.path.join(HERE, "golden", "q4_0_ref.npz"))
    table = g["blocks"].reshape(31, 16 * 18)  # 496 blocks = 31 rows of 512 values
    ids = np.arange(30, -1, -1, dtype=np.int32)
    got = host(jinf_amd.embed_q4_0(to_dev(table), to_dev(ids), 512, torch.float16))
    ref32 = g["out"].reshape(31, 512)[ids]
    with np.errstate(over="ignore", invalid="ignore"):
        assert tu.bits_equal(got, ref32.astype(np.float16))


def test_config4_full_size_bit_exact(dev):
    say("config 4: table 128256x4096, 4096 ids, fp16 and fp32 out")
    r = tu.rng(4)
    n_vocab, n_embd = 128256, 4096
    table = tu.q4_0_table(r, n_vocab, n_embd)
    ids = r.integers(0, n_vocab, size=4096).astype(np.int32)
    t_dev, i_dev = to_dev(table), to_dev(ids)
    ref = oracle.embed_q4_0(table, ids, n_embd, np.float16)
    got = host(jinf_amd.embed_q4_0(t_dev, i_dev, n_embd, torch.float16))
    assert tu.bits_equal(got, ref)
    ref32 = oracle.embed_q4_0(table, ids, n_embd, np.float32)
    got32 = host(jinf_amd.embed_q4_0(t_dev, i_dev, n_embd, torch.float32))
    assert tu.bits_equal(got32, ref32)


def test_llama70b_rows_and_bad_ids(dev):
    say("70B rows (8192 values), ids outside [0, n_vocab) give +0 rows")
    r = tu.rng(7)
    table = tu.q4_0_table(r, 300, 8192)
    ids = r.integers(-5, 305, size=257).astype(np.int32)
    for dt, ndt in ((torch.float16, np.float16), (torch.float32, np.float32)):
        got = host(jinf_amd.embed_q4_0(to_dev(table), to_dev(ids), 8192, dt))
        assert tu.bits_equal(got, oracle.embed_q4_0(table, ids, 8192, ndt))


def test_identity_rows_without_ids(dev):
    say("ids = NULL: rows 0..n-1")
    r = tu.rng(9)
    table = tu.q4_0_table(r, 64, 2048)
    got = host(jinf_amd.embed_q4_0(to_dev(table), None, 2048, torch.float16))
    assert tu.bits_equal(got, oracle.embed_q4_0(table, None, 2048, np.float16))


@pytest.mark.parametrize("n_embd,offset", [(4096, 0), (32 * 129, 0), (32 * 130, 0),
                                           (4096, 2), (4096, 1), (32 * 3, 4),
                                           (32 * 1100, 0), (32 * 1100, 1)])
def test_staging_width_paths(dev, n_embd, offset):
    say(f"n_embd={n_embd}, table byte offset {offset}")
    r = tu.rng(8)
    table = tu.q4_0_table(r, 40, n_embd)
    blk = table.reshape(-1, 18)
    sel = blk[::7]
    sel[:, 0:2] = r.integers(0, 65536, size=(sel.shape[0], 1), dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blk[::7] = sel
    ids = r.integers(0, 40, size=23).astype(np.int32)
    raw = np.zeros(table.size + 64, np.uint8)
    raw[offset:offset + table.size] = table.reshape(-1)
    buf, ids_d = to_dev(raw), to_dev(ids)
    L = jinf_amd.lib()
    for dt, ndt, code in ((torch.float16, np.float16, 1), (torch.float32, np.float32, 0)):
        out = torch.empty((23, n_embd), dtype=dt, device=dev)
        rc = L.jinf_embed_q4_0(ctypes.c_void_p(out.data_ptr()), n_embd,
                               ctypes.c_void_p(buf.data_ptr() + offset), 40, n_embd,
                               ctypes.c_void_p(ids_d.data_ptr()), 23, code, _stream())
        assert rc == 0
        with np.errstate(over="ignore", invalid="ignore"):
            assert tu.bits_equal(host(out), oracle.embed_q4_0(table, ids, n_embd, ndt))


@pytest.mark.parametrize("n_blocks,in_off,out_off", [(1, 0, 0), (3, 2, 1), (128, 0, 0),
                                                     (127, 18, 3), (513, 1, 0), (1025, 0, 2),
                                                     (4096 * 32, 0, 0)])
def test_drop_in_any_alignment(dev, n_blocks, in_off, out_off):
    say(f"drop-in dequant n_blocks={n_blocks} data+{in_off} out+{out_off} floats")
    r = tu.rng(10)
    blocks = tu.q4_0_table(r, 1, n_blocks * 32).reshape(-1)
    raw = np.zeros(blocks.size + 32, np.uint8)
    raw[in_off:in_off + blocks.size] = blocks
    buf = to_dev(raw)
    out = torch.full((n_blocks * 32 + 8,), -1.0, dtype=torch.float32, device=dev)
    jinf_amd.lib().jinf_cuda_dequantize_q4_0(ctypes.c_void_p(buf.data_ptr() + in_off),
                                             ctypes.c_void_p(out.data_ptr() + 4 * out_off),
                                             n_blocks, _stream())
    o = host(out)
    assert tu.bits_equal(o[out_off:out_off + n_blocks * 32], oracle.dequant_q4_0(blocks))
    assert np.all(o[:out_off] == -1.0) and np.all(o[out_off + n_blocks * 32:] == -1.0)
