""".nvmw model files through libjinf_hip.so (include/jinf/nvmw_hip.h): header,
layer cold ranges, tensor entries and tensor upload into device memory."""
import ctypes

from ._lib import JINF_HIP_OK, lib


class Header(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_uint32), ("version", ctypes.c_uint32),
                ("n_layers", ctypes.c_uint32), ("n_tensors", ctypes.c_uint32),
                ("index_offset", ctypes.c_uint64), ("index_size", ctypes.c_uint64),
                ("hot_offset", ctypes.c_uint64), ("hot_size", ctypes.c_uint64),
                ("cold_start_offset", ctypes.c_uint64), ("cold_total_size", ctypes.c_uint64),
                ("n_embd", ctypes.c_uint32), ("n_heads", ctypes.c_uint32),
                ("n_heads_kv", ctypes.c_uint32), ("n_ff", ctypes.c_uint32),
                ("n_vocab", ctypes.c_uint32), ("n_ctx_train", ctypes.c_uint32),
                ("rope_freq_base", ctypes.c_float), ("rms_norm_eps", ctypes.c_float),
                ("primary_type", ctypes.c_int32), ("bundle_index_offset", ctypes.c_uint64)]


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("qtype", ctypes.c_int),
                ("shape", ctypes.c_int64 * 4), ("n_dims", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("n_bytes", ctypes.c_uint64),
                ("layer_index", ctypes.c_int32), ("is_hot", ctypes.c_int),
                ("file_offset", ctypes.c_uint64)]


class NVMWError(RuntimeError):
    pass


class NVMWFile:
    """A parsed .nvmw file (jinf_hip_nvmw_load); close() frees it."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        rc = lib().jinf_hip_nvmw_load(ctypes.byref(h), str(path).encode())
        if rc != JINF_HIP_OK:
            raise NVMWError(f"jinf_hip_nvmw_load({path}) returned status {rc}")
        self._h = h

    def close(self):
        if self._h:
            lib().jinf_hip_nvmw_free(self._h)
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

    @property
    def header(self):
        h = Header.from_address(lib().jinf_hip_nvmw_header_of(self._h))
        return {f: getattr(h, f) for f, _ in Header._fields_}

    def tensor_count(self):
        return lib().jinf_hip_nvmw_n_tensors(self._h)

    def tensor(self, i):
        t = Tensor.from_address(lib().jinf_hip_nvmw_tensor_at(self._h, i))
        return {"name": t.name.decode(), "qtype": t.qtype, "shape": list(t.shape),
                "n_dims": t.n_dims, "offset": t.offset, "n_bytes": t.n_bytes,
                "layer_index": t.layer_index, "is_hot": t.is_hot,
                "file_offset": t.file_offset}

    def find_tensor(self, name):
        return lib().jinf_hip_nvmw_find_tensor(self._h, name.encode())

    def layer_cold_range(self, layer):
        off, size = ctypes.c_uint64(), ctypes.c_uint64()
        rc = lib().jinf_hip_nvmw_layer_cold_range(self._h, layer, ctypes.byref(off),
                                                  ctypes.byref(size))
        if rc != JINF_HIP_OK:
            raise NVMWError(f"jinf_hip_nvmw_layer_cold_range({layer}) returned status {rc}")
        return off.value, size.value

    def has_bundles(self):
        return bool(lib().jinf_hip_nvmw_has_bundles(self._h))

    def upload(self, i, dst, stream=None):
        """Copy tensor i's bytes into the device tensor dst (>= n_bytes)."""
        import torch
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().jinf_hip_nvmw_upload(self._h, i, ctypes.c_void_p(dst.data_ptr()),
                                        dst.numel() * dst.element_size(), ctypes.c_void_p(s))
        if rc != JINF_HIP_OK:
            raise NVMWError(f"jinf_hip_nvmw_upload returned status {rc}")
        return dst
