""".nvmw reader (include/jinf/nvmw_hip.h) on the CPU: field-by-field agreement
with the reference reader itself (src/nvmw.cpp, compiled into oracle/_ref) on
files laid out as prepare_model writes them -- every tensor hot, some layers
cold, a version-2 file with neuron bundles, a tied output, a version number
the reader does not know -- plus the resolved absolute offsets checked against
the bytes in the file, the bundle-index corner cases and the files both
readers reject.  Deliberate difference: an index entry whose data lies past
the end of the file (or a cold entry without a layer descriptor) is a parse
error here, where the reference accepts the file and would read out of range
later."""
import ctypes
import struct

import numpy as np
import pytest

import model_util as mu
import nvmw_writer as nw
import oracle
from jinf_amd.nvmw import NVMWError, NVMWFile


def _dump(path):
    """This repository's reader, printed in the reference shim's format."""
    with NVMWFile(path) as f:
        h = f.header
        lines = ["header %d %d %d %d %d %d %d %d %d %d" % tuple(
                     h[k] for k in ("magic", "version", "n_layers", "n_tensors", "index_offset",
                                    "index_size", "hot_offset", "hot_size", "cold_start_offset",
                                    "cold_total_size")),
                 "hparams %d %d %d %d %d %d %.9g %.9g %d %d" % tuple(
                     h[k] for k in ("n_embd", "n_heads", "n_heads_kv", "n_ff", "n_vocab",
                                    "n_ctx_train", "rope_freq_base", "rms_norm_eps",
                                    "primary_type", "bundle_index_offset"))]
        for L in range(h["n_layers"]):
            lines.append("layer %d %d %d" % ((L,) + f.layer_cold_range(L)))
        for i in range(f.tensor_count()):
            t = f.tensor(i)
            lines.append("tensor %s %d %d %d %d %d %d %d %d %d %d" % (
                t["name"], t["qtype"], *t["shape"], t["n_dims"], t["offset"], t["n_bytes"],
                t["layer_index"], t["is_hot"]))
        lines.append("bundles %d" % f.has_bundles())
    return "\n".join(lines) + "\n"


def _ref_dump(path):
    buf = ctypes.create_string_buffer(1 << 20)
    ref = oracle.ref()
    ref.jref_nvmw_dump.restype = ctypes.c_int
    ref.jref_nvmw_dump.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
    st = ref.jref_nvmw_dump(str(path).encode(), buf, len(buf))
    return st, buf.value.decode()


def _need_ref():
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built")


CASES = {
    "all-hot": dict(),
    "layer1-cold": dict(cold_layers=(1,)),
    "all-cold": dict(cold_layers=(0, 1, 2)),
    "bundled": dict(cold_layers=(2,), bundled=True),
}


def _model(tied=False):
    return mu.tiny_model(seed=31, n_layers=3, n_embd=256, n_ff=512, n_vocab=300, tied=tied)


@pytest.mark.parametrize("case", list(CASES))
def test_agrees_with_reference_reader(tmp_path, case):
    _need_ref()
    hp, W = _model()
    p = tmp_path / "m.nvmw"
    mu.write_nvmw(str(p), hp, W, **CASES[case])
    st, ref = _ref_dump(p)
    assert st == 0
    assert _dump(p) == ref
    assert ("bundles 1" in ref) == (case == "bundled")


def test_unknown_version_and_tied_output_agree(tmp_path):
    _need_ref()
    hp, W = _model(tied=True)
    p = tmp_path / "m.nvmw"
    mu.write_nvmw(str(p), hp, W, cold_layers=(0,))
    b = bytearray(p.read_bytes())
    struct.pack_into("<I", b, 4, 77)   # only the magic is checked
    p.write_bytes(bytes(b))
    st, ref = _ref_dump(p)
    assert st == 0 and _dump(p) == ref
    with NVMWFile(p) as f:
        assert f.header["version"] == 77 and f.find_tensor("output.weight") == -1


def test_offsets_resolve_to_the_tensor_bytes(tmp_path):
    hp, W = _model()
    p = tmp_path / "m.nvmw"
    h = mu.write_nvmw(str(p), hp, W, cold_layers=(1, 2), bundled=True)
    raw = p.read_bytes()
    with NVMWFile(p) as f:
        assert f.tensor_count() == len(W) == h["n_tensors"]
        assert f.has_bundles() and f.header["version"] == 2
        for name, (a, qt) in W.items():
            i = f.find_tensor(name)
            t = f.tensor(i)
            assert t["name"] == name and t["qtype"] == qt
            base = h["hot_offset"] if t["is_hot"] else f.layer_cold_range(t["layer_index"])[0]
            assert t["file_offset"] == base + t["offset"]
            assert t["file_offset"] % 4096 == 0
            data = np.ascontiguousarray(a).tobytes()
            assert t["n_bytes"] == len(data)
            assert raw[t["file_offset"]:t["file_offset"] + len(data)] == data, name
            assert t["is_hot"] == (not name.startswith(("blk.1.", "blk.2.")))
            assert t["shape"][:t["n_dims"]] == mu.gguf_shape(hp, name, a)
        with pytest.raises(NVMWError):
            f.layer_cold_range(3)
        with pytest.raises(NVMWError):
            f.layer_cold_range(-1)
        assert f.find_tensor("blk.9.attn_q.weight") == -1


def test_bundle_index_corner_cases(tmp_path):
    """A bundle offset past the end, or a truncated layer list, leaves the
    file readable without bundles (src/nvmw.cpp:232-255)."""
    hp, W = _model()
    p = tmp_path / "m.nvmw"
    h = mu.write_nvmw(str(p), hp, W, bundled=True)
    good = p.read_bytes()
    for name, edit in (("past-end", lambda b: struct.pack_into("<Q", b, 104, len(b) + 4096)),
                       ("truncated", lambda b: b.__delitem__(slice(len(b) - 10, None))),
                       ("too-many-layers",
                        lambda b: struct.pack_into("<I", b, h["bundle_index_offset"], 1000))):
        b = bytearray(good)
        edit(b)
        p.write_bytes(bytes(b))
        with NVMWFile(p) as f:
            assert not f.has_bundles(), name
        if oracle.ref_available():
            st, ref = _ref_dump(p)
            assert st == 0 and ref.endswith("bundles 0\n"), name


def test_rejected_files(tmp_path):
    hp, W = _model()
    p = tmp_path / "m.nvmw"
    h = mu.write_nvmw(str(p), hp, W, cold_layers=(2,))
    good = p.read_bytes()

    def variant(edit):
        b = bytearray(good)
        edit(b)
        p.write_bytes(bytes(b))
        return p

    both = {  # the reference rejects these too
        "bad-magic": lambda b: struct.pack_into("<I", b, 0, 0x46554747),
        "short-header": lambda b: b.__delitem__(slice(100, None)),
        "index-past-end": lambda b: struct.pack_into("<Q", b, 16, len(b) - 100),
        "too-many-tensors": lambda b: struct.pack_into("<I", b, 12, 100000),
    }
    for name, edit in both.items():
        variant(edit)
        with pytest.raises(NVMWError, match="status 2"):
            NVMWFile(p)
        if oracle.ref_available():
            assert _ref_dump(p)[0] == 2, name
    e0 = h["index_offset"] + h["n_layers"] * nw.LAYER_BYTES
    only_here = {
        "data-past-end": lambda b: struct.pack_into("<Q", b, e0 + 184, len(b)),
        "cold-without-layer": lambda b: struct.pack_into(
            "<i", b, e0 + (h["n_tensors"] - 1) * nw.ENTRY_BYTES + 192, 7),
    }
    for name, edit in only_here.items():
        variant(edit)
        with pytest.raises(NVMWError, match="status 2"):
            NVMWFile(p)
    with pytest.raises(NVMWError, match="status 1"):
        NVMWFile(tmp_path / "missing.nvmw")
