"""ctypes binding of libjinf_hip.so, the C-ABI declared in include/jinf/*.h.

The library links the HIP runtime by soname (libamdhip64.so.7).  PyTorch ships
its own copy with the same soname, so torch is imported first: the dynamic
loader then resolves the library's HIP dependency to the runtime torch already
loaded, and device pointers and streams from torch are valid in both.

There is no fallback: if the shared library is missing, `lib()` raises.
"""
import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libjinf_hip.so")

JINF_HIP_OK = 0
JINF_HIP_ERR_DEVICE = 3
JINF_HIP_ERR_INVALID = 5

F32 = 0
F16 = 1

# GGUF block codes (jinf_qtype values)
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); the parameter lists of the C declarations.
SIGNATURES = {
    # drop-ins (include/jinf/kernels.h)
    "jinf_cuda_rmsnorm": (None, [_P, _P, _P, _I, _F, _I, _P]),
    "jinf_cuda_rope": (None, [_P, _P, _I, _I, _I, _I, _F, _P]),
    "jinf_cuda_silu_mul": (None, [_P, _P, _P, _I, _P]),
    "jinf_cuda_softmax": (None, [_P, _P, _I, _P]),
    "jinf_cuda_residual_add": (None, [_P, _P, _I, _P]),
    "jinf_cuda_dequantize_q4_0": (None, [_P, _P, _I, _P]),
    "jinf_cuda_dequant_matvec": (None, [_P, _P, _P, _I, _I, _I, _P]),
    "jinf_cuda_dequantize_q4_K": (None, [_P, _P, _I, _P]),
    "jinf_cuda_dequantize_q8_0": (None, [_P, _P, _I, _P]),
    "jinf_cuda_dequantize_q6_K": (None, [_P, _P, _I, _P]),
    "jinf_cuda_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    # extensions (include/jinf/kernels_ext.h)
    "jinf_hip_version": (ctypes.c_char_p, []),
    "jinf_rmsnorm_rows": (_I, [_P, _I, _P, _I, _P, _I, _I, _F, _I, _I, _P]),
    "jinf_residual_rmsnorm_rows": (_I, [_P, _I, _P, _I, _P, _I, _P, _I, _I, _F, _I, _I, _P]),
    "jinf_rope_rows": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _F, _I, _P]),
    "jinf_swiglu_rows": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P]),
    "jinf_residual_add_rows": (_I, [_P, _I, _P, _I, _I, _I, _I, _P]),
    "jinf_softmax_rows_f32": (_I, [_P, _I, _P, _I, _I, _I, _P, _I, _F, _P]),
    "jinf_embed_q4_0": (_I, [_P, _I, _P, _I, _I, _P, _I, _I, _P]),
    "jinf_matvec_q4_0": (_I, [_P, _P, _P, _I, _I, _P]),
    "jinf_matvec": (_I, [_P, _I, _P, _P, _I, _I, _P]),
    "jinf_dequant_rows": (_I, [_P, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "jinf_attention_decode": (_I, [_P, _I, _P, _I, _P, _P, _I, ctypes.c_int64, ctypes.c_int64,
                                   _P, _I, _I, _I, _I, _I, _F, _P, ctypes.c_size_t, _P]),
    "jinf_attention_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I, _I]),
    "jinf_attention_decode_noalloc": (_I, [_P, _I, _P, _I, _P, _P, _I, ctypes.c_int64,
                                           ctypes.c_int64, _P, _I, _I, _I, _I, _I, _F, _P]),
    "jinf_rmsnorm_matvec": (_I, [_P, _I, _P, _P, _I, _F, _P, _I, _I, _P]),
    "jinf_matvec_add": (_I, [_P, _I, _P, _P, _I, _I, _P]),
    "jinf_rmsnorm_swiglu_matvec": (_I, [_P, _P, _I, _P, _P, _I, _F, _P, _I, _I, _P]),
    "jinf_rmsnorm_qkv_rope": (_I, [_P, _P, _P, _I, _P, _P, _I, _F, _I, _P, _P, _P, _I, _P, _I,
                                   _I, _I, _I, _F, _P]),
    # batched GEMVs on the matrix cores
    "jinf_matvec_batch_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I]),
    "jinf_matvec_batch": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P]),
    "jinf_matvec_batch_add": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, ctypes.c_size_t,
                                   _P]),
    "jinf_rmsnorm_matvec_batch": (_I, [_P, _I, _P, _I, _P, _I, _F, _P, _I, _I, _I, _I, _P,
                                       ctypes.c_size_t, _P]),
    "jinf_rmsnorm_swiglu_matvec_batch": (_I, [_P, _P, _I, _P, _I, _P, _I, _F, _P, _I, _I, _I,
                                              _I, _P, ctypes.c_size_t, _P]),
    "jinf_rmsnorm_qkv_rope_batch": (_I, [_P, _P, _P, _I, _P, _I, _P, _I, _F, _I, _P, _I, _P,
                                         _P, _I, ctypes.c_int64, _P, _I, _I, _I, _I, _F, _I,
                                         _P, ctypes.c_size_t, _P]),
    # bandwidth probes (include/jinf/probe_hip.h)
    "jinf_probe_rows_inplace": (_I, [_P, ctypes.c_int64, _I, _P, ctypes.c_int64, _I, _I, _I,
                                     _I, _P]),
    "jinf_probe_stream": (_I, [_P, _P, _P, _P, ctypes.c_int64, _I, _I, _P]),
    "jinf_probe_stream_layout": (_I, [_P, _P, _P, _P, ctypes.c_int64, _I, _I, _I, _I, _P]),
    "jinf_probe_read_layout": (_I, [_P, ctypes.c_int64, _P, _I, _I, _I, _P]),
    "jinf_probe_gather": (_I, [_P, ctypes.c_int64, _I, _P, ctypes.c_int64, _I, _I, _P, _I, _I,
                               _I, _P]),
    "jinf_probe_rows_ragged": (_I, [_P, ctypes.c_int64, _P, ctypes.c_int64, _I, _P, _I, _I,
                                    _P]),
    # GGUF files (include/jinf/gguf_hip.h)
    "jinf_hip_gguf_load": (_I, [ctypes.POINTER(_P), ctypes.c_char_p]),
    "jinf_hip_gguf_free": (None, [_P]),
    "jinf_hip_gguf_version": (ctypes.c_uint32, [_P]),
    "jinf_hip_gguf_alignment": (ctypes.c_uint32, [_P]),
    "jinf_hip_gguf_data_offset": (ctypes.c_uint64, [_P]),
    "jinf_hip_gguf_n_kv": (ctypes.c_uint64, [_P]),
    "jinf_hip_gguf_n_tensors": (ctypes.c_uint64, [_P]),
    "jinf_hip_gguf_hparams_of": (_P, [_P]),
    "jinf_hip_gguf_find_kv": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "jinf_hip_gguf_kv_key": (ctypes.c_char_p, [_P, ctypes.c_uint64]),
    "jinf_hip_gguf_kv_type": (_I, [_P, ctypes.c_uint64]),
    "jinf_hip_gguf_kv_scalar": (_I, [_P, ctypes.c_uint64, _P]),
    "jinf_hip_gguf_kv_str": (ctypes.c_char_p, [_P, ctypes.c_uint64]),
    "jinf_hip_gguf_kv_array": (_I, [_P, ctypes.c_uint64, ctypes.POINTER(_I),
                                    ctypes.POINTER(ctypes.c_uint64)]),
    "jinf_hip_gguf_get_str": (ctypes.c_char_p, [_P, ctypes.c_char_p, ctypes.c_char_p]),
    "jinf_hip_gguf_get_u32": (ctypes.c_uint32, [_P, ctypes.c_char_p, ctypes.c_uint32]),
    "jinf_hip_gguf_get_f32": (_F, [_P, ctypes.c_char_p, _F]),
    "jinf_hip_gguf_find_tensor": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "jinf_hip_gguf_tensor_at": (_P, [_P, ctypes.c_uint64]),
    "jinf_hip_gguf_upload": (_I, [_P, ctypes.c_uint64, _P, ctypes.c_uint64, _P]),
    "jinf_hip_q4_0_repack_ggml": (_I, [_P, ctypes.c_int64, _P]),
    # .nvmw files (include/jinf/nvmw_hip.h)
    "jinf_hip_nvmw_load": (_I, [ctypes.POINTER(_P), ctypes.c_char_p]),
    "jinf_hip_nvmw_free": (None, [_P]),
    "jinf_hip_nvmw_header_of": (_P, [_P]),
    "jinf_hip_nvmw_n_tensors": (ctypes.c_uint64, [_P]),
    "jinf_hip_nvmw_tensor_at": (_P, [_P, ctypes.c_uint64]),
    "jinf_hip_nvmw_find_tensor": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "jinf_hip_nvmw_layer_cold_range": (_I, [_P, _I, ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_uint64)]),
    "jinf_hip_nvmw_has_bundles": (_I, [_P]),
    "jinf_hip_nvmw_upload": (_I, [_P, ctypes.c_uint64, _P, ctypes.c_uint64, _P]),
    # decode engine (include/jinf/engine_hip.h)
    "jinf_hip_engine_create": (_I, [ctypes.POINTER(_P), _P]),
    "jinf_hip_engine_create_gguf": (_I, [ctypes.POINTER(_P), _P, _I, _I, _I]),
    "jinf_hip_engine_create_nvmw": (_I, [ctypes.POINTER(_P), _P, _I, _I]),
    "jinf_hip_engine_destroy": (None, [_P]),
    "jinf_hip_engine_reset": (_I, [_P]),
    "jinf_hip_engine_n_past": (_I, [_P]),
    "jinf_hip_engine_forward": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "jinf_hip_engine_prefill": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "jinf_hip_engine_generate": (_I, [_P, _P, _I, _P, _I, ctypes.POINTER(_I)]),
    "jinf_hip_engine_copy_logits": (_I, [_P, _P, _I]),
    "jinf_hip_engine_use_graph": (_I, [_P, _I]),
    "jinf_hip_engine_step_weight_bytes": (ctypes.c_uint64, [_P]),
    "jinf_hip_engine_get_stats": (_P, [_P]),
    # the reference's engine API by name (include/jinf/engine_api.h)
    "jinf_engine_create": (_I, [ctypes.POINTER(_P), _P]),
    "jinf_engine_destroy": (None, [_P]),
    "jinf_engine_forward": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "jinf_engine_generate": (_I, [_P, _P, _I, _P, _I, ctypes.POINTER(_I)]),
    "jinf_engine_reset": (None, [_P]),
    "jinf_engine_get_stats": (_P, [_P]),
    # batched decode (include/jinf/engine_hip.h)
    "jinf_hip_batch_create": (_I, [ctypes.POINTER(_P), _P, _I, _I, _I]),
    "jinf_hip_batch_destroy": (None, [_P]),
    "jinf_hip_batch_reset": (_I, [_P, _I]),
    "jinf_hip_batch_n_past": (_I, [_P, _I]),
    "jinf_hip_batch_forward": (_I, [_P, _P, ctypes.POINTER(_P)]),
    "jinf_hip_batch_prefill": (_I, [_P, _I, _P, _I, ctypes.POINTER(_P)]),
    "jinf_hip_batch_generate": (_I, [_P, _P, _I]),
    "jinf_hip_batch_copy_logits": (_I, [_P, _P]),
    "jinf_hip_batch_use_graph": (_I, [_P, _I]),
}

_lib = None


def lib():
    """Load libjinf_hip.so (after torch) and declare every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (must precede the load; see module docstring)

    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `make -C jetson-inference_amd`")
    handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return _lib


def version():
    return lib().jinf_hip_version().decode()
