"""GGUF reader (include/jinf/gguf_hip.h) on the CPU: the reference's own test
case as known answers (tests/test_gguf.cpp:36-126), and field-by-field
agreement with the reference reader itself (src/gguf.cpp, compiled into
oracle/_ref) on synthetic files covering every value type, nested arrays,
alignment overrides, version 2, every tensor type and the hyper-parameter
defaults and conversions.  Malformed files give status 2 (parse)."""
import ctypes
import os

import numpy as np
import pytest

import jinf_amd
import oracle
from jinf_amd.gguf import GGUFError, GGUFFile

import gguf_writer as gw


def _dump(path):
    """This repository's reader, printed in the reference shim's format."""
    with GGUFFile(path) as f:
        lines = [f"version {f.version}", f"alignment {f.alignment}",
                 f"data_offset {f.data_offset}", f"kv_count {f.kv_count()}",
                 f"tensor_count {f.tensor_count()}"]
        for i in range(f.kv_count()):
            key, t, v = f.kv(i)
            if t == gw.F32:
                vs = "%.9g" % v
            elif t == gw.F64:
                vs = "%.17g" % v
            elif t == gw.BOOL:
                vs = str(int(v))
            elif t == gw.ARR:
                vs = "[%d x %d]" % v
            else:
                vs = str(v)
            lines.append(f"kv {key} {t} {vs}")
        for i in range(f.tensor_count()):
            t = f.tensor(i)
            dims = "".join(f" {d}" for d in t["shape"])
            lines.append(f"tensor {t['name']} {t['n_dims']}{dims} type {t['qtype']} offset "
                         f"{t['offset']} n_elements {t['n_elements']} n_bytes {t['n_bytes']}")
        h = f.hparams
        lines.append("hparams %s %d %d %d %d %d %d %d %.9g %.9g" % (
            h["arch"], h["n_layers"], h["n_embd"], h["n_heads"], h["n_heads_kv"], h["n_ff"],
            h["n_vocab"], h["n_ctx_train"], h["rope_freq_base"], h["rms_norm_eps"]))
    return "\n".join(lines) + "\n"


def _ref_dump(path):
    buf = ctypes.create_string_buffer(1 << 20)
    ref = oracle.ref()
    ref.jref_gguf_dump.restype = ctypes.c_int
    ref.jref_gguf_dump.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
    st = ref.jref_gguf_dump(str(path).encode(), buf, len(buf))
    return st, buf.value.decode()


def _reference_test_file(path):
    """The synthetic file of the reference's tests/test_gguf.cpp:36-80."""
    kvs = [("general.architecture", gw.STR, "llama"), ("llama.block_count", gw.U32, 2),
           ("llama.embedding_length", gw.U32, 64), ("llama.attention.head_count", gw.U32, 4),
           ("llama.attention.layer_norm_rms_epsilon", gw.F32, 1e-5)]
    tensors = [("token_embd.weight", [64, 100], 2, bytes(6400 // 32 * 18))]
    return gw.write(path, kvs, tensors)


def test_reference_test_case_known_answers(tmp_path):
    p = tmp_path / "test_jinf.gguf"
    _reference_test_file(p)
    with GGUFFile(p) as f:
        assert f.version == 3 and f.tensor_count() == 1 and f.kv_count() == 5
        h = f.hparams
        assert (h["n_layers"], h["n_embd"], h["n_heads"], h["arch"]) == (2, 64, 4, "llama")
        assert f.kv(f.find_kv("llama.block_count"))[2] == 2
        assert f.get_u32("llama.embedding_length", 0) == 64
        t = f.tensor(0)
        assert t["n_dims"] == 2 and t["shape"] == [64, 100] and t["qtype"] == 2
        assert t["n_elements"] == 6400
        assert f.tensor(f.find_tensor("token_embd.weight"))["shape"][0] == 64
        assert f.find_kv("nonexistent") == -1 and f.find_tensor("nonexistent") == -1
        # defaults the reference applies (src/gguf.cpp:279-303)
        assert h["n_heads_kv"] == 4 and h["n_ctx_train"] == 2048 and h["n_vocab"] == 100
        assert h["rope_freq_base"] == 10000.0 and h["rms_norm_eps"] == np.float32(1e-5)
    with pytest.raises(GGUFError):
        GGUFFile(tmp_path / "nonexistent_file.gguf")


def _all_types_file(path, version=3, alignment=None):
    kvs = [("general.architecture", gw.STR, "llama"),
           ("general.name", gw.STR, "synthetic model"),
           ("llama.block_count", gw.U32, 32), ("llama.embedding_length", gw.I32, 4096),
           ("llama.attention.head_count", gw.U64, 32),
           ("llama.attention.head_count_kv", gw.I64, 8),
           ("llama.feed_forward_length", gw.F32, 14336.0),
           ("llama.context_length", gw.U32, 8192),
           ("llama.rope.freq_base", gw.F64, 500000.0),
           ("llama.attention.layer_norm_rms_epsilon", gw.F32, 1e-5),
           ("t.u8", gw.U8, 250), ("t.i8", gw.I8, -7), ("t.u16", gw.U16, 65000),
           ("t.i16", gw.I16, -30000), ("t.bool", gw.BOOL, True), ("t.neg_i32", gw.I32, -5),
           ("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["<s>", "</s>", "hello", ""])),
           ("tokenizer.ggml.scores", gw.ARR, (gw.F32, [0.5, -1.25, 3.0])),
           ("t.nested", gw.ARR, (gw.ARR, [(gw.U8, [1, 2, 3]), (gw.STR, ["a", "bc"])])),
           ("t.empty", gw.ARR, (gw.I64, []))]
    if alignment is not None:
        kvs.append(("general.alignment", gw.U32, alignment))
    tensors = [("token_embd.weight", [4096, 300], 2, gw.random_bytes(1, 4096 * 300 // 32 * 18)),
               ("blk.0.attn_norm.weight", [4096], 0, gw.random_bytes(2, 4096 * 4)),
               ("blk.0.ffn_down.weight", [14336, 16], 14, gw.random_bytes(3, 14336 * 16 // 256 * 210)),
               ("blk.0.attn_q.weight", [256, 8], 12, gw.random_bytes(4, 256 * 8 // 256 * 144)),
               ("blk.0.attn_v.weight", [64, 3], 8, gw.random_bytes(5, 64 * 3 // 32 * 34)),
               ("output.weight", [7, 5], 1, gw.random_bytes(6, 7 * 5 * 2)),
               ("odd.type", [10], 99, bytes(40))]  # unknown type code: read as F32 (0)
    return gw.write(path, kvs, tensors, version=version, alignment=alignment)


@pytest.mark.parametrize("version,alignment", [(3, None), (2, None), (3, 64), (3, 4096)])
def test_agrees_with_reference_reader(tmp_path, version, alignment):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    p = tmp_path / "m.gguf"
    _all_types_file(p, version, alignment)
    st, ref = _ref_dump(p)
    assert st == 0
    assert _dump(p) == ref


def test_hparams_defaults_and_conversions(tmp_path):
    p = tmp_path / "m.gguf"
    _all_types_file(p)
    with GGUFFile(p) as f:
        h = f.hparams
        assert (h["n_layers"], h["n_embd"], h["n_heads"], h["n_heads_kv"], h["n_ff"]) == (32, 4096, 32, 8, 14336)
        assert h["n_ctx_train"] == 8192 and h["rope_freq_base"] == 500000.0
        assert h["n_vocab"] == 300  # from token_embd.weight's second dimension
        assert f.get_u32("t.neg_i32", 1) == 2**32 - 5       # (uint32_t) of an int32
        assert f.get_f32("t.neg_i32", 0.0) == -5.0
        assert f.get_u32("t.u8", 9) == 9                     # u8 is not converted
        assert f.get_str("general.name") == "synthetic model"
        assert f.get_str("llama.block_count", "x") == "x"    # not a string
        assert f.kv(f.find_kv("t.nested"))[2] == (gw.ARR, 2)
        assert f.tensor(f.find_tensor("odd.type"))["qtype"] == 0


@pytest.mark.parametrize("damage", ["magic", "version", "truncated", "string_len", "n_dims",
                                    "alignment0", "data_past_end", "bad_type", "negative_dim",
                                    "dims_overflow", "bytes_past_end", "offset_wraps"])
def test_malformed_files_are_parse_errors(tmp_path, damage):
    p = tmp_path / "bad.gguf"
    kvs = [("general.architecture", gw.STR, "llama")]
    tensors = [("t", [32, 1], 2, bytes(18))]
    if damage == "alignment0":
        kvs.append(("general.alignment", gw.U32, 0))
    if damage == "bad_type":
        kvs.append(("x", gw.U8, 1))
    data_offset = gw.write(p, kvs, tensors)
    b = bytearray(open(p, "rb").read())
    # tensor "t": n_dims (u32) at i, dims (i64) at i + 4 and i + 12, type at
    # i + 20, offset (u64) at i + 24
    i = b.index(b"\x01\x00\x00\x00\x00\x00\x00\x00t") + 9
    if damage == "magic":
        b[0] = ord("X")
    elif damage == "version":
        b[4] = 4
    elif damage == "truncated":
        b = b[:40]
    elif damage == "string_len":
        b[24:32] = (2 << 20).to_bytes(8, "little")  # first key longer than 1 MiB
    elif damage == "n_dims":
        b[i:i + 4] = (5).to_bytes(4, "little")
    elif damage == "negative_dim":
        b[i + 4:i + 12] = (-32).to_bytes(8, "little", signed=True)
    elif damage == "dims_overflow":  # 2^62 x 4 elements: the product passes int64
        b[i + 4:i + 12] = (1 << 62).to_bytes(8, "little")
        b[i + 12:i + 20] = (4).to_bytes(8, "little")
    elif damage == "bytes_past_end":  # 2^60 elements fit, their bytes do not
        b[i + 4:i + 12] = (1 << 60).to_bytes(8, "little")
    elif damage == "offset_wraps":  # data_offset + offset fits, + n_bytes wraps to 17
        b[i + 24:i + 32] = ((1 << 64) - data_offset - 1).to_bytes(8, "little")
    elif damage == "data_past_end":
        b = b[:-1]
    elif damage == "bad_type":
        i = b.index(b"x") + 1
        b[i:i + 4] = (13).to_bytes(4, "little")  # value type 13 does not exist
    open(p, "wb").write(bytes(b))
    h = ctypes.c_void_p()
    rc = jinf_amd.lib().jinf_hip_gguf_load(ctypes.byref(h), str(p).encode())
    assert rc == 2 and not h.value


def test_upload_and_repack_reject_bad_arguments():
    L = jinf_amd.lib()
    assert L.jinf_hip_gguf_upload(None, 0, ctypes.c_void_p(16), 16, None) == 5
    assert L.jinf_hip_q4_0_repack_ggml(None, 4, None) == 5
    assert L.jinf_hip_q4_0_repack_ggml(None, 0, None) == 0
