"""GPU: GGUF tensor upload into device memory (bytes identical to the file,
across the 32 MiB staging chunks) and the Q4_0 element-order conversion for
upstream-ggml files: a table written in upstream order, uploaded and
repacked, then gathered by jinf_embed_q4_0, equals the upstream dequantization
restated in numpy (element j: low nibble of qs[j], element j + 16: its high
nibble; value (q - 8) * d) -- parity pinned by this restatement and by the
order-independence checks (constant nibbles, one-hot nibble positions)."""
import numpy as np
import pytest
import torch

import jinf_amd
import oracle
import testutil as tu
from gpu_util import host, say
from jinf_amd.gguf import GGUFFile, q4_0_repack_ggml

import gguf_writer as gw

pytestmark = pytest.mark.gpu


def ggml_order_dequant(blocks):
    b = blocks.reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    qs = b[:, 2:].astype(np.int32)
    out = np.empty((b.shape[0], 32), np.float32)
    out[:, :16] = ((qs & 0x0F) - 8).astype(np.float32) * d[:, None]
    out[:, 16:] = ((qs >> 4) - 8).astype(np.float32) * d[:, None]
    return out.reshape(-1)


def test_upload_bytes_across_chunks(dev, tmp_path):
    say("GGUF upload: 3 tensors, one spanning 4 staging chunks")
    sizes = [(100 << 20) + 18, 4096 * 4, 1000]
    data = [gw.random_bytes(10 + i, n) for i, n in enumerate(sizes)]
    # F32 tensors of n/4 elements hold exactly their bytes
    tensors = [(f"t{i}", [len(d) // 4], 0, d[: len(d) // 4 * 4]) for i, d in enumerate(data)]
    p = tmp_path / "u.gguf"
    gw.write(p, [("general.alignment", gw.U32, 64)], tensors, alignment=64)
    with GGUFFile(p) as f:
        for i, (_, _, _, d) in enumerate(tensors):
            dst = torch.empty(len(d) + 7, dtype=torch.uint8, device=dev)
            dst.fill_(0xAB)
            f.upload(i, dst)
            h = host(dst)
            assert h[:len(d)].tobytes() == d, i
            assert np.all(h[len(d):] == 0xAB)


def test_upstream_q4_0_table_repack_and_gather(dev, tmp_path):
    say("upstream-order Q4_0 table: upload, repack, gather == ggml-order dequant")
    n_vocab, n_embd = 500, 4096
    r = tu.rng(21)
    table = tu.q4_0_table(r, n_vocab, n_embd, 0.05)
    p = tmp_path / "m.gguf"
    gw.write(p, [("general.architecture", gw.STR, "llama")],
             [("token_embd.weight", [n_embd, n_vocab], 2, table.tobytes())])
    with GGUFFile(p) as f:
        i = f.find_tensor("token_embd.weight")
        t = f.tensor(i)
        assert t["n_bytes"] == table.size
        dev_t = torch.empty((n_vocab, n_embd // 32 * 18), dtype=torch.uint8, device=dev)
        f.upload(i, dev_t)
    q4_0_repack_ggml(dev_t)
    ids = np.array([0, 499, 7, 123, 7], np.int32)
    out = host(jinf_amd.embed_q4_0(dev_t, torch.from_numpy(ids).to(dev), n_embd, torch.float32))
    want = ggml_order_dequant(table).reshape(n_vocab, n_embd)
    assert tu.bits_equal(out, want[ids])


def test_repack_nibble_positions(dev):
    say("repack: each upstream nibble position lands on its element")
    blocks = np.zeros((32, 18), np.uint8)
    blocks[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    for e in range(32):  # block e: element e has q = 9 (value 1), every other q = 8 (value 0)
        blocks[e, 2:] = 0x88
        j = e % 16
        blocks[e, 2 + j] = (0x89 if e < 16 else 0x98)
    d = torch.from_numpy(blocks.reshape(-1).copy()).to(dev)
    q4_0_repack_ggml(d)
    vals = oracle.dequant_q4_0(host(d)).reshape(32, 32)
    assert np.array_equal(vals, np.eye(32, dtype=np.float32))
