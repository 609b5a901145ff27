"""GPU: .nvmw tensor upload into device memory (hot and cold tensors, bytes
identical to the file) and the decode engine built from a .nvmw file
(jinf_hip_engine_create_nvmw) -- the same logits, bit for bit, as the engine
built from the same weights already resident, whichever layers the file keeps
cold, with a neuron-bundle index present, a tied output and a file whose
entries are in a different order; the engine from resident weights is itself
pinned against the oracle's decode loop in test_gpu_engine.py.  Missing or
misshapen tensors are rejected with status 2 / 5."""
import struct

import numpy as np
import pytest
import torch

import model_util as mu
import nvmw_writer as nw
from gpu_util import host, say
from jinf_amd.engine import Engine, EngineError
from jinf_amd.nvmw import NVMWFile

pytestmark = pytest.mark.gpu

TOKENS = [5, 17, 299, 0, 42, 17, 3, 200]


def test_upload_hot_and_cold(dev, tmp_path):
    say("NVMW upload: every tensor of a 3-layer file with layer 1 cold")
    hp, W = mu.tiny_model(seed=41, n_layers=3, n_vocab=300)
    p = tmp_path / "m.nvmw"
    mu.write_nvmw(str(p), hp, W, cold_layers=(1,))
    with NVMWFile(p) as f:
        for name, (a, _) in W.items():
            i = f.find_tensor(name)
            data = np.ascontiguousarray(a).tobytes()
            dst = torch.empty(len(data) + 5, dtype=torch.uint8, device=dev)
            dst.fill_(0xCD)
            f.upload(i, dst)
            h = host(dst)
            assert h[:len(data)].tobytes() == data, name
            assert np.all(h[len(data):] == 0xCD), name


VARIANTS = {
    "all-hot": (dict(), dict()),
    "cold-layers-bundled": (dict(), dict(cold_layers=(0, 2), bundled=True)),
    "tied-f16norm": (dict(tied=True, norm_type=mu.F16, embd_type=mu.Q4_0), dict(cold_layers=(1,))),
    "reordered": (dict(), "reverse"),
}


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_engine_from_nvmw_matches_resident_weights(dev, tmp_path, variant):
    say(f"engine from a .nvmw file: {variant}")
    model_kw, file_kw = VARIANTS[variant]
    hp, W = mu.tiny_model(seed=42, n_layers=3, n_vocab=300, **model_kw)
    p = tmp_path / "m.nvmw"
    if file_kw == "reverse":
        mu.write_nvmw(str(p), hp, W, cold_layers=(1,), order=list(reversed(list(W))))
    else:
        mu.write_nvmw(str(p), hp, W, **file_kw)
    with Engine(hp, mu.to_device(W), 16, mu.F16) as a, Engine.from_nvmw(str(p), 16, mu.F16) as b:
        assert b.step_weight_bytes == a.step_weight_bytes
        for tok in TOKENS:
            a.forward([tok])
            b.forward([tok])
            assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32)), tok
        out_a, out_b = a.generate([], 6), b.generate([], 6)
        assert out_a == out_b


def test_nvmw_missing_or_misshapen_tensor(dev, tmp_path):
    hp, W = mu.tiny_model(seed=43, n_layers=2, n_vocab=300)
    p = tmp_path / "broken.nvmw"
    W2 = dict(W)
    del W2["blk.1.attn_v.weight"]
    mu.write_nvmw(str(p), hp, W2, cold_layers=(1,))
    with pytest.raises(EngineError) as ex:
        Engine.from_nvmw(str(p), 16)
    assert ex.value.status == 2
    # n_ff in the header disagrees with the FFN matrices
    h = mu.write_nvmw(str(p), hp, W)
    b = bytearray(p.read_bytes())
    struct.pack_into("<I", b, 76, hp["n_ff"] * 2)
    p.write_bytes(bytes(b))
    with pytest.raises(EngineError) as ex:
        Engine.from_nvmw(str(p), 16)
    assert ex.value.status == 5
    assert h["n_tensors"] == len(W) and nw.MAGIC == h["magic"]
