"""GGUF model files through libjinf_hip.so (include/jinf/gguf_hip.h): metadata,
tensor upload into device memory, and the Q4_0 element-order conversion for
files written by upstream ggml."""
import ctypes

from ._lib import JINF_HIP_OK, lib

# GGUF value types
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: ctypes.c_uint8, INT8: ctypes.c_int8, UINT16: ctypes.c_uint16,
           INT16: ctypes.c_int16, UINT32: ctypes.c_uint32, INT32: ctypes.c_int32,
           FLOAT32: ctypes.c_float, BOOL: ctypes.c_bool, UINT64: ctypes.c_uint64,
           INT64: ctypes.c_int64, FLOAT64: ctypes.c_double}


class Hparams(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_char * 64), ("n_layers", ctypes.c_uint32),
                ("n_embd", ctypes.c_uint32), ("n_heads", ctypes.c_uint32),
                ("n_heads_kv", ctypes.c_uint32), ("n_ff", ctypes.c_uint32),
                ("n_vocab", ctypes.c_uint32), ("n_ctx_train", ctypes.c_uint32),
                ("rope_freq_base", ctypes.c_float), ("rms_norm_eps", ctypes.c_float)]


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_int64 * 4), ("qtype", ctypes.c_int),
                ("offset", ctypes.c_uint64), ("n_elements", ctypes.c_int64),
                ("n_bytes", ctypes.c_uint64)]


class GGUFError(RuntimeError):
    pass


class GGUFFile:
    """A parsed GGUF file (jinf_hip_gguf_load); close() frees it."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        rc = lib().jinf_hip_gguf_load(ctypes.byref(h), str(path).encode())
        if rc != JINF_HIP_OK:
            raise GGUFError(f"jinf_hip_gguf_load({path}) returned status {rc}")
        self._h = h

    def close(self):
        if self._h:
            lib().jinf_hip_gguf_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # header
    @property
    def version(self):
        return lib().jinf_hip_gguf_version(self._h)

    @property
    def alignment(self):
        return lib().jinf_hip_gguf_alignment(self._h)

    @property
    def data_offset(self):
        return lib().jinf_hip_gguf_data_offset(self._h)

    @property
    def hparams(self):
        p = lib().jinf_hip_gguf_hparams_of(self._h)
        hp = Hparams.from_address(p)
        return {f: (getattr(hp, f).decode() if f == "arch" else getattr(hp, f))
                for f, _ in Hparams._fields_}

    # key/value pairs
    def kv_count(self):
        return lib().jinf_hip_gguf_n_kv(self._h)

    def kv(self, i):
        """(key, type, value); arrays give (elem_type, count)."""
        L = lib()
        key = L.jinf_hip_gguf_kv_key(self._h, i).decode()
        t = L.jinf_hip_gguf_kv_type(self._h, i)
        if t == STRING:
            return key, t, L.jinf_hip_gguf_kv_str(self._h, i).decode()
        if t == ARRAY:
            et, n = ctypes.c_int(), ctypes.c_uint64()
            L.jinf_hip_gguf_kv_array(self._h, i, ctypes.byref(et), ctypes.byref(n))
            return key, t, (et.value, n.value)
        v = _SCALAR[t]()
        L.jinf_hip_gguf_kv_scalar(self._h, i, ctypes.byref(v))
        return key, t, v.value

    def find_kv(self, key):
        return lib().jinf_hip_gguf_find_kv(self._h, key.encode())

    def get_str(self, key, default=None):
        d = None if default is None else default.encode()
        r = lib().jinf_hip_gguf_get_str(self._h, key.encode(), d)
        return None if r is None else r.decode()

    def get_u32(self, key, default=0):
        return lib().jinf_hip_gguf_get_u32(self._h, key.encode(), default)

    def get_f32(self, key, default=0.0):
        return lib().jinf_hip_gguf_get_f32(self._h, key.encode(), default)

    # tensors
    def tensor_count(self):
        return lib().jinf_hip_gguf_n_tensors(self._h)

    def tensor(self, i):
        t = Tensor.from_address(lib().jinf_hip_gguf_tensor_at(self._h, i))
        return {"name": t.name.decode(), "n_dims": t.n_dims,
                "shape": list(t.shape[:t.n_dims]), "qtype": t.qtype, "offset": t.offset,
                "n_elements": t.n_elements, "n_bytes": t.n_bytes}

    def find_tensor(self, name):
        return lib().jinf_hip_gguf_find_tensor(self._h, name.encode())

    def upload(self, i, dst, stream=None):
        """Copy tensor i's bytes into the device tensor dst (uint8, >= n_bytes)."""
        import torch
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().jinf_hip_gguf_upload(self._h, i, ctypes.c_void_p(dst.data_ptr()),
                                        dst.numel() * dst.element_size(), ctypes.c_void_p(s))
        if rc != JINF_HIP_OK:
            raise GGUFError(f"jinf_hip_gguf_upload returned status {rc}")
        return dst


def q4_0_repack_ggml(blocks, n_blocks=None):
    """In place: upstream-ggml Q4_0 element order -> jinf's (device uint8 tensor)."""
    import torch
    n = blocks.numel() // 18 if n_blocks is None else n_blocks
    rc = lib().jinf_hip_q4_0_repack_ggml(ctypes.c_void_p(blocks.data_ptr()), n,
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if rc != JINF_HIP_OK:
        raise GGUFError(f"jinf_hip_q4_0_repack_ggml returned status {rc}")
    return blocks
