"""GPU: .nvmw tensor upload into device memory (hot and cold tensors, bytes
identical to the file) and the decode engine built from a .nvmw file
(jinf_hip_engine_create_nvmw) -- the same logits, bit for bit, as the engine
built from the same weights already resident, whichever layers the file keeps
cold, with a neuron-bundle index present, a tied output and a file whose
entries are in a different order; the engine from resident weights is itself
pinned against the oracle's decode loop in test_gpu_engine.py.  Missing or
misshapen tensors are rejected with status 2 / 5."""
import ctypes
import struct

import numpy as np
import pytest
import torch

import model_util as mu
import nvmw_writer as nw
from gpu_util import host, say
from jinf_amd import lib
from jinf_amd.engine import Engine, EngineError, PerfStats
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


class EngineConfig(ctypes.Structure):
    """jinf_engine_config (include/jinf/engine_api.h), the reference's layout."""
    _fields_ = [("model_path", ctypes.c_char_p), ("gpu_memory_budget", ctypes.c_size_t),
                ("buffer_capacity", ctypes.c_size_t), ("max_context", ctypes.c_int),
                ("io_queue_depth", ctypes.c_int), ("predictor_path", ctypes.c_char_p),
                ("sparsity_threshold", ctypes.c_float)]


def device_floats(ptr, n):
    out = np.empty(n, np.float32)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(out.ctypes.data, ctypes.c_void_p(ptr), out.nbytes, 4) == 0  # default
    return out


def test_reference_engine_api(dev, tmp_path):
    """include/jinf/engine_api.h: the reference's jinf_engine_create / forward /
    generate / reset / get_stats (include/jinf/engine.h:159-176) over a .nvmw
    file give the logits and tokens of jinf_hip_engine_create_nvmw with an fp32
    cache, bit for bit, and the reference's counters; a sparse-FFN predictor is
    rejected (5)."""
    say("reference-named engine API against jinf_hip_engine_create_nvmw (fp32 cache)")
    hp, W = mu.tiny_model(seed=44, n_layers=2, n_vocab=300)
    p = tmp_path / "m.nvmw"
    mu.write_nvmw(str(p), hp, W, cold_layers=(1,))
    L = lib()
    h = ctypes.c_void_p()
    bad = EngineConfig(str(p).encode(), 4500 << 20, 128 << 20, 16, 64, b"pred.bin", 0.5)
    assert L.jinf_engine_create(ctypes.byref(h), ctypes.byref(bad)) == 5 and not h.value
    cfg = EngineConfig(str(p).encode(), 4500 << 20, 128 << 20, 16, 64, None, 0.5)
    assert L.jinf_engine_create(ctypes.byref(h), ctypes.byref(cfg)) == 0
    try:
        with Engine.from_nvmw(str(p), 16, mu.F32) as ref:
            for tok in TOKENS[:5]:
                t = (ctypes.c_int32 * 1)(tok)
                lg = ctypes.c_void_p()
                assert L.jinf_engine_forward(h, t, 1, ctypes.byref(lg)) == 0
                ref.forward([tok])
                got = device_floats(lg.value, hp["n_vocab"])
                assert np.array_equal(got.view(np.uint32), ref.logits().view(np.uint32)), tok
            out = (ctypes.c_int32 * 6)()
            n = ctypes.c_int()
            assert L.jinf_engine_generate(h, None, 0, out, 6, ctypes.byref(n)) == 0
            assert list(out[:n.value]) == ref.generate([], 6)
            st = PerfStats.from_address(L.jinf_engine_get_stats(h))
            assert st.tokens_generated == 5 + (n.value - (1 if out[n.value - 1] == 2 else 0))
            assert st.total_ms > 0.0 and st.nvme_bytes_read == 0.0
            L.jinf_engine_reset(h)
            st = PerfStats.from_address(L.jinf_engine_get_stats(h))
            assert st.tokens_generated == 0 and st.total_ms == 0.0
            # after a reset the first token decodes as from a fresh engine
            ref.reset()
            t = (ctypes.c_int32 * 2)(7, 9)
            lg = ctypes.c_void_p()
            assert L.jinf_engine_forward(h, t, 2, ctypes.byref(lg)) == 0
            ref.forward([7, 9])
            got = device_floats(lg.value, hp["n_vocab"])
            assert np.array_equal(got.view(np.uint32), ref.logits().view(np.uint32))
    finally:
        L.jinf_engine_destroy(h)
    assert L.jinf_engine_get_stats(None) is None
