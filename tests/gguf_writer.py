"""Writes GGUF files for the tests (format of the reference reader,
src/gguf.cpp:143-311): header, key/value pairs of every value type
(arrays included), tensor infos, alignment padding and tensor data."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write(path, kvs, tensors, version=3, alignment=None, pad_value=0):
    """kvs: [(key, type, value)]; tensors: [(name, shape, ggml_type, data bytes)].
    Tensor offsets are assigned consecutively, each aligned; returns the
    absolute data offset."""
    align = alignment if alignment is not None else 32
    out = bytearray(struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kvs)))
    for key, t, v in kvs:
        out += _str(key) + struct.pack("<I", t) + _value(t, v)
    off = 0
    offsets = []
    for name, shape, gtype, data in tensors:
        off = (off + align - 1) // align * align
        offsets.append(off)
        out += _str(name) + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<q", d) for d in shape)
        out += struct.pack("<IQ", gtype, off)
        off += len(data)
    data_offset = (len(out) + align - 1) // align * align
    out += bytes([pad_value]) * (data_offset - len(out))
    for (name, shape, gtype, data), o in zip(tensors, offsets):
        out += bytes(data_offset + o - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)
    return data_offset


def random_bytes(seed, n):
    return np.random.default_rng(seed).integers(0, 256, size=n, dtype=np.uint8).tobytes()
