"""The C-ABI boundary without a GPU: libjinf_hip.so loads, exports every entry
point include/jinf/*.h declares with the declared arity, and rejects bad
arguments on the host (status JINF_HIP_ERR_INVALID) before any HIP call."""
import ctypes
import os
import re

import pytest

import jinf_amd
from jinf_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "jinf", h)
           for h in sorted(os.listdir(os.path.join(ROOT, "include", "jinf"))) if h.endswith(".h")]


def declared():
    """{name: n_params} for every function declared in the public headers."""
    out = {}
    for h in HEADERS:
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\b(jinf_\w+)\s*\(([^)]*)\)\s*;", src):
            params = m.group(2).strip()
            n = 0 if params in ("", "void") else params.count(",") + 1
            out[m.group(1)] = n
    return out


def test_headers_include_no_gpu_runtime_header():
    for h in HEADERS:
        src = open(h).read()
        assert "cuda" not in re.findall(r"#include\s*[<\"]([^>\"]+)", src.lower())
        assert not re.search(r"#include\s*[<\"](hip|cuda)", src)


def test_every_declared_symbol_is_exported_with_declared_arity():
    decl = declared()
    assert len(decl) == 99
    lib = jinf_amd.lib()
    for name, n in decl.items():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_version():
    assert "gfx950" in jinf_amd.version()


P = ctypes.c_void_p
FAKE = P(0x1000)  # never dereferenced: every call below is rejected on the host


@pytest.mark.parametrize("call", [
    lambda L: L.jinf_rmsnorm_rows(FAKE, 64, FAKE, 64, FAKE, -1, 64, 1e-5, 1, 1, None),
    lambda L: L.jinf_rmsnorm_rows(FAKE, 64, FAKE, 64, FAKE, 4, 64, 1e-5, 7, 1, None),
    lambda L: L.jinf_rmsnorm_rows(FAKE, 64, FAKE, 64, FAKE, 4, 64, 1e-5, 1, 9, None),
    lambda L: L.jinf_rmsnorm_rows(FAKE, 32, FAKE, 64, FAKE, 4, 64, 1e-5, 1, 1, None),
    lambda L: L.jinf_rmsnorm_rows(None, 64, FAKE, 64, FAKE, 4, 64, 1e-5, 1, 1, None),
    lambda L: L.jinf_residual_rmsnorm_rows(FAKE, 64, FAKE, 64, FAKE, 64, FAKE, 4, 64, 1e-5, 1, 1, None),
    lambda L: L.jinf_rope_rows(FAKE, 256, FAKE, 128, None, 0, 4, 127, 2, 1, 1e4, 1, None),
    lambda L: L.jinf_rope_rows(FAKE, 2048, FAKE, 1024, None, 0, 4, 1024, 2, 1, 1e4, 1, None),
    lambda L: L.jinf_rope_rows(FAKE, 100, FAKE, 128, None, 0, 4, 128, 2, 1, 1e4, 1, None),
    lambda L: L.jinf_swiglu_rows(FAKE, 64, FAKE, 64, FAKE, 32, 2, 64, 1, None),
    lambda L: L.jinf_swiglu_rows(FAKE, 64, FAKE, 64, FAKE, 64, 2, 64, 3, None),
    lambda L: L.jinf_residual_add_rows(FAKE, 64, None, 64, 2, 64, 1, None),
    lambda L: L.jinf_softmax_rows_f32(FAKE, 64, FAKE, 64, 2, 64, None, 1, 0.0, None, 0, None),
    lambda L: L.jinf_softmax_rows_f32(FAKE, 64, FAKE, 64, 2, 64, FAKE, 0, 1.0, None),
    lambda L: L.jinf_softmax_rows_f32(FAKE, 64, FAKE, 64, 2, 64, None, 1, float("nan"), None),
    lambda L: L.jinf_embed_q4_0(FAKE, 100, FAKE, 10, 100, FAKE, 4, 1, None),
    lambda L: L.jinf_embed_q4_0(FAKE, 128, FAKE, 10, 128, FAKE, 4, 2, None),
    lambda L: L.jinf_embed_q4_0(FAKE, 128, FAKE, 10, 128, None, 11, 1, None),
    lambda L: L.jinf_matvec_q4_0(FAKE, FAKE, FAKE, 16, 100, None),
    lambda L: L.jinf_matvec_q4_0(FAKE, FAKE, FAKE, -1, 128, None),
    lambda L: L.jinf_matvec_q4_0(None, FAKE, FAKE, 16, 128, None),
    lambda L: L.jinf_matvec(FAKE, 3, FAKE, FAKE, 16, 128, None),     # Q4_1: not served
    lambda L: L.jinf_matvec(FAKE, 12, FAKE, FAKE, 16, 128, None),    # Q4_K needs cols % 256
    lambda L: L.jinf_matvec(FAKE, 14, FAKE, FAKE, 16, 4097, None),
    lambda L: L.jinf_dequant_rows(FAKE, 256, FAKE, 3, 10, 256, FAKE, 4, 0, None),
    lambda L: L.jinf_dequant_rows(FAKE, 128, FAKE, 12, 10, 128, FAKE, 4, 0, None),
    lambda L: L.jinf_dequant_rows(FAKE, 100, FAKE, 8, 10, 128, FAKE, 4, 0, None),
    lambda L: L.jinf_dequant_rows(FAKE, 256, FAKE, 14, 10, 256, None, 11, 0, None),
    # attention: lens missing, n_heads not a multiple of n_heads_kv, bad scale,
    # ld_pos below one position, kv type, head_dim too large
    lambda L: L.jinf_attention_decode(FAKE, 256, FAKE, 256, FAKE, FAKE, 0, 128, 4096, None, 2, 32, 128, 2, 1, 0.0, None, 0, None),
    lambda L: L.jinf_attention_decode(FAKE, 384, FAKE, 384, FAKE, FAKE, 0, 256, 8192, FAKE, 2, 32, 128, 3, 2, 0.0, None, 0, None),
    lambda L: L.jinf_attention_decode(FAKE, 256, FAKE, 256, FAKE, FAKE, 0, 128, 4096, FAKE, 2, 32, 128, 2, 1, -1.0, None, 0, None),
    lambda L: L.jinf_attention_decode(FAKE, 256, FAKE, 256, FAKE, FAKE, 0, 64, 4096, FAKE, 2, 32, 128, 2, 1, 0.0, None, 0, None),
    lambda L: L.jinf_attention_decode(FAKE, 256, FAKE, 256, FAKE, FAKE, 7, 128, 4096, FAKE, 2, 32, 128, 2, 1, 0.0, None, 0, None),
    lambda L: L.jinf_attention_decode(FAKE, 4096, FAKE, 4096, FAKE, FAKE, 0, 2048, 65536, FAKE, 2, 32, 2048, 2, 1, 0.0, None, 0, None),
    # fused GEMVs: qtype, whole blocks, norm type, missing operands, head_dim,
    # kv type, missing position
    lambda L: L.jinf_rmsnorm_matvec(FAKE, 3, FAKE, FAKE, 0, 1e-5, FAKE, 16, 256, None),
    lambda L: L.jinf_rmsnorm_matvec(FAKE, 12, FAKE, FAKE, 0, 1e-5, FAKE, 16, 128, None),
    lambda L: L.jinf_rmsnorm_matvec(FAKE, 2, FAKE, FAKE, 2, 1e-5, FAKE, 16, 256, None),
    lambda L: L.jinf_rmsnorm_matvec(FAKE, 2, FAKE, FAKE, 0, -1.0, FAKE, 16, 256, None),
    lambda L: L.jinf_matvec_add(None, 2, FAKE, FAKE, 16, 256, None),
    lambda L: L.jinf_rmsnorm_swiglu_matvec(FAKE, None, 2, FAKE, FAKE, 0, 1e-5, FAKE, 16, 256, None),
    lambda L: L.jinf_rmsnorm_qkv_rope(FAKE, FAKE, FAKE, 2, FAKE, FAKE, 0, 1e-5, 256, FAKE, FAKE, FAKE, 1, FAKE, 64, 63, 4, 2, 1e4, None),
    lambda L: L.jinf_rmsnorm_qkv_rope(FAKE, FAKE, FAKE, 2, FAKE, FAKE, 0, 1e-5, 256, FAKE, FAKE, FAKE, 5, FAKE, 64, 64, 4, 2, 1e4, None),
    lambda L: L.jinf_rmsnorm_qkv_rope(FAKE, FAKE, FAKE, 2, FAKE, FAKE, 0, 1e-5, 256, FAKE, FAKE, FAKE, 1, None, 64, 64, 4, 2, 1e4, None),
    lambda L: L.jinf_rmsnorm_qkv_rope(FAKE, FAKE, FAKE, 2, FAKE, FAKE, 0, 1e-5, 256, None, FAKE, FAKE, 1, FAKE, 64, 64, 4, 2, 1e4, None),
    lambda L: L.jinf_rmsnorm_qkv_rope(FAKE, FAKE, FAKE, 2, FAKE, FAKE, 0, 1e-5, 256, FAKE, FAKE, FAKE, 1, FAKE, 64, 64, 4, 2, 0.0, None),
])
def test_invalid_arguments_rejected_on_host(call):
    assert call(jinf_amd.lib()) == _lib.JINF_HIP_ERR_INVALID


@pytest.mark.parametrize("call", [
    lambda L: L.jinf_rmsnorm_rows(FAKE, 64, FAKE, 64, FAKE, 0, 64, 1e-5, 1, 1, None),
    lambda L: L.jinf_swiglu_rows(FAKE, 64, FAKE, 64, FAKE, 64, 2, 0, 1, None),
    lambda L: L.jinf_rope_rows(FAKE, 256, FAKE, 128, None, 0, 0, 128, 2, 1, 1e4, 1, None),
    lambda L: L.jinf_softmax_rows_f32(FAKE, 64, FAKE, 64, 0, 64, None, 1, 1.0, None),
    lambda L: L.jinf_embed_q4_0(FAKE, 128, FAKE, 10, 128, FAKE, 0, 1, None),
    lambda L: L.jinf_matvec_q4_0(FAKE, FAKE, FAKE, 0, 128, None),
    lambda L: L.jinf_matvec(FAKE, 14, FAKE, FAKE, 16, 0, None),
    lambda L: L.jinf_dequant_rows(FAKE, 256, FAKE, 12, 10, 256, FAKE, 0, 0, None),
    lambda L: L.jinf_attention_decode(FAKE, 256, FAKE, 256, FAKE, FAKE, 0, 128, 4096, FAKE, 0, 32, 128, 2, 1, 0.0, None, 0, None),
])
def test_empty_work_is_ok_and_enqueues_nothing(call):
    assert call(jinf_amd.lib()) == _lib.JINF_HIP_OK


def test_drop_ins_are_noops_for_empty_sizes():
    L = jinf_amd.lib()
    L.jinf_cuda_rmsnorm(FAKE, FAKE, FAKE, 0, 1e-5, 0, None)
    L.jinf_cuda_softmax(FAKE, FAKE, -5, None)
    L.jinf_cuda_silu_mul(FAKE, FAKE, FAKE, 0, None)
    L.jinf_cuda_residual_add(FAKE, FAKE, 0, None)
    L.jinf_cuda_dequantize_q4_0(FAKE, FAKE, 0, None)
    L.jinf_cuda_rope(FAKE, FAKE, 128, 0, 0, 5, 1e4, None)
    L.jinf_cuda_dequant_matvec(FAKE, FAKE, FAKE, 0, 128, 2, None)
    L.jinf_cuda_dequant_matvec(FAKE, FAKE, FAKE, 16, 128, 3, None)  # unsupported qtype: no-op
    L.jinf_cuda_dequantize_q4_K(FAKE, FAKE, 0, None)
    L.jinf_cuda_dequantize_q8_0(FAKE, FAKE, -1, None)
    L.jinf_cuda_dequantize_q6_K(FAKE, FAKE, 0, None)
    L.jinf_cuda_attention(FAKE, FAKE, FAKE, FAKE, 128, 32, 8, 0, 4096, None)
