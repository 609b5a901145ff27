"""CPU oracle for jinf's per-layer elementwise / reduction kernels.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product path never imports
it.

numpy front end over libjinf_oracle.so (jinf_oracle.c, a C restatement of the
reference arithmetic; each function there cites the reference file:line it
follows) and, when built, _ref/libjinf_ref.so (the reference's own
src/quant.cpp compiled in place, used to pin the Q4_0 and fp16 restatement).
fp16 arrays are numpy float16 (IEEE binary16).
"""
import ctypes
import os

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))


def _has_avx512():
    """x86-64-v4's AVX-512 subsets (F, BW, CD, DQ, VL) on this host."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= fl
    except OSError:
        pass
    return False


# the AVX-512 build where the host has it and it was built, else the AVX2 one
ORACLE_PATH = os.path.join(_DIR, "libjinf_oracle_v4.so")
if not (_has_avx512() and os.path.exists(ORACLE_PATH)):
    ORACLE_PATH = os.path.join(_DIR, "libjinf_oracle.so")
REF_PATH = os.path.join(_DIR, "_ref", "libjinf_ref.so")

F32, F16 = 0, 1

_P, _I, _F, _L = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_int64
_SIG = {
    "jo_set_threads": (None, [_I]),
    "jo_get_threads": (_I, []),
    "jo_f16_to_f32": (_F, [ctypes.c_uint16]),
    "jo_f32_to_f16": (ctypes.c_uint16, [_F]),
    "jo_f16_to_f32_n": (None, [_P, _P, _L]),
    "jo_f32_to_f16_n": (None, [_P, _P, _L]),
    "jo_dequant_q4_0": (None, [_P, _P, _I]),
    "jo_embed_q4_0": (None, [_P, _I, _L, _P, _I, _I, _P, _I]),
    "jo_rmsnorm_rows": (None, [_P, _L, _P, _L, _P, _I, _I, _F, _I, _I]),
    "jo_residual_rmsnorm_rows": (None, [_P, _L, _P, _L, _P, _L, _P, _I, _I, _F, _I, _I]),
    "jo_ref_order_sumsq": (_F, [_P, _I]),
    "jo_residual_add": (None, [_P, _P, _L, _I]),
    "jo_rope_theta": (_F, [_F, _I, _I]),
    "jo_rope_rows": (None, [_P, _L, _P, _L, _P, _I, _I, _I, _I, _I, _F, _I]),
    "jo_swiglu": (None, [_P, _P, _P, _L, _I]),
    "jo_softmax_rows": (None, [_P, _L, _P, _L, _I, _I, _P, _I, _F]),
    "jo_matvec_q4_0": (None, [_P, _P, _P, _P, _I, _I]),
    "jo_qtype_geometry": (_I, [_I, ctypes.POINTER(_I)]),
    "jo_dequant": (None, [_I, _P, _P, _I]),
    "jo_matvec": (None, [_I, _P, _P, _P, _P, _I, _I]),
    "jo_attention": (None, [_P, _L, _P, _L, _P, _P, _I, _L, _L, _P, _I, _I, _I, _I,
                            ctypes.c_double, _P]),
}

# qtype codes (include/jinf/quant.h:8-24)
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} not built (make -C oracle)")
        h = ctypes.CDLL(ORACLE_PATH)
        for n, (r, a) in _SIG.items():
            f = getattr(h, n)
            f.restype, f.argtypes = r, a
        _lib = h
    return _lib


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own CPU routines (src/quant.cpp), or None if not built."""
    global _ref
    if _ref is None and ref_available():
        h = ctypes.CDLL(REF_PATH)
        h.jref_dequantize_q4_0.restype = None
        h.jref_dequantize_q4_0.argtypes = [_P, _P, _I]
        h.jref_f16_to_f32.restype = None
        h.jref_f16_to_f32.argtypes = [_P, _P, ctypes.c_longlong]
        for n in ("jref_dequantize_q4_K", "jref_dequantize_q8_0"):
            getattr(h, n).restype = None
            getattr(h, n).argtypes = [_P, _P, _I]
        _ref = h
    return _ref


def set_threads(n):
    lib().jo_set_threads(int(n))


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _act(a):
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise TypeError(a.dtype)


def _c(a):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a


# ---- conversions ----

def f16_to_f32(h):
    h = _c(np.asarray(h, dtype=np.float16))
    out = np.empty(h.shape, np.float32)
    lib().jo_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f32_to_f16(x):
    x = _c(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.float16)
    lib().jo_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


# ---- Q4_0 ----

def dequant_q4_0(blocks_u8):
    """Contiguous Q4_0 blocks (uint8, 18 bytes each) -> fp32 (src/quant.cpp:49-60)."""
    b = _c(np.asarray(blocks_u8, dtype=np.uint8)).reshape(-1)
    nb = b.size // 18
    out = np.empty(nb * 32, np.float32)
    lib().jo_dequant_q4_0(_p(b), _p(out), nb)
    return out


def ref_dequant_q4_0(blocks_u8):
    """Same, through the reference's own compiled jinf_dequantize_q4_0."""
    b = _c(np.asarray(blocks_u8, dtype=np.uint8)).reshape(-1)
    nb = b.size // 18
    out = np.empty(nb * 32, np.float32)
    ref().jref_dequantize_q4_0(_p(b), _p(out), nb)
    return out


def ref_f16_to_f32(h):
    h = _c(np.asarray(h, dtype=np.float16))
    out = np.empty(h.shape, np.float32)
    ref().jref_f16_to_f32(_p(h), _p(out), h.size)
    return out


def embed_q4_0(table_u8, ids, n_embd, out_dtype=np.float16):
    """table: uint8 [n_vocab, n_embd/32*18]; ids int32 [n] (None = every row)."""
    t = _c(np.asarray(table_u8, dtype=np.uint8))
    n_vocab = t.shape[0]
    ids_a = None if ids is None else _c(np.asarray(ids, dtype=np.int32))
    n = n_vocab if ids_a is None else ids_a.shape[0]
    out = np.empty((n, n_embd), out_dtype)
    lib().jo_embed_q4_0(_p(out), _act(out), n_embd, _p(t), n_vocab, n_embd, _p(ids_a), n)
    return out


# ---- RMSNorm / residual ----

def rmsnorm_rows(x, w, eps):
    x = _c(x)
    w = _c(w)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    assert n <= 65536
    out = np.empty_like(x)
    lib().jo_rmsnorm_rows(_p(out), n, _p(x), n, _p(w), rows, n, float(eps), _act(x), _act(w))
    return out


def residual_rmsnorm_rows(res, delta, w, eps):
    """Returns (new_residual, out) without modifying the inputs."""
    r = _c(res).copy()
    d = _c(delta)
    w = _c(w)
    rows, n = r.reshape(-1, r.shape[-1]).shape
    assert n <= 65536
    out = np.empty_like(r)
    lib().jo_residual_rmsnorm_rows(_p(out), n, _p(r), n, _p(d), n, _p(w), rows, n, float(eps),
                                   _act(r), _act(w))
    return r, out


def ref_order_sumsq(x):
    x = _c(np.asarray(x, dtype=np.float32))
    return lib().jo_ref_order_sumsq(_p(x), x.size)


def residual_add(a, b):
    r = _c(a).copy()
    lib().jo_residual_add(_p(r), _p(_c(b)), r.size, _act(r))
    return r


# ---- RoPE ----

def rope_theta(base, i, head_dim):
    return lib().jo_rope_theta(float(base), int(i), int(head_dim))


def rope_rows(q, k, head_dim, positions=None, pos0=0, base=10000.0):
    """q [T, nh*hd], k [T, nkv*hd] -> rotated copies."""
    q2 = _c(q).copy()
    k2 = _c(k).copy()
    T = q2.shape[0]
    pos = None if positions is None else _c(np.asarray(positions, dtype=np.int32))
    nh = q2.reshape(T, -1).shape[1] // head_dim
    nkv = k2.reshape(T, -1).shape[1] // head_dim
    lib().jo_rope_rows(_p(q2), nh * head_dim, _p(k2), nkv * head_dim, _p(pos), int(pos0), T,
                       head_dim, nh, nkv, float(base), _act(q2))
    return q2, k2


# ---- SwiGLU ----

def swiglu(gate, up):
    g = _c(gate)
    out = np.empty_like(g)
    lib().jo_swiglu(_p(out), _p(g), _p(_c(up)), g.size, _act(g))
    return out


# ---- softmax ----

def softmax_rows(x, lens=None, rows_per_len=1, scale=1.0, out=None):
    """x fp32 [rows, n_cols]; rows j >= len keep `out`'s prior content."""
    x = _c(np.asarray(x, dtype=np.float32))
    rows, n = x.shape
    out = x.copy() if out is None else _c(out).copy()
    l_a = None if lens is None else _c(np.asarray(lens, dtype=np.int32))
    lib().jo_softmax_rows(_p(out), n, _p(x), n, rows, n, _p(l_a), int(rows_per_len),
                          float(scale))
    return out


# ---- Q4_0 dequant-GEMV ----

def matvec_q4_0(W_u8, x):
    """W uint8 [rows, cols/32*18] Q4_0, x fp32 [cols] -> (y fp32 [rows],
    sum_j |w_j x_j| fp64 [rows])."""
    W = _c(np.asarray(W_u8, dtype=np.uint8))
    x = _c(np.asarray(x, dtype=np.float32))
    rows = W.shape[0]
    cols = x.shape[0]
    assert W.shape[1] == cols // 32 * 18
    y = np.empty(rows, np.float32)
    a = np.empty(rows, np.float64)
    lib().jo_matvec_q4_0(_p(W), _p(x), _p(y), _p(a), rows, cols)
    return y, a


# ---- Q8_0 / Q4_K / Q6_K ----

def qtype_geometry(qtype):
    """(values per block, bytes per block) of a supported qtype, else (0, 0)."""
    b = _I(0)
    e = lib().jo_qtype_geometry(int(qtype), ctypes.byref(b))
    return e, b.value


def dequant(qtype, blocks_u8):
    """Contiguous blocks of qtype (uint8) -> fp32 values."""
    e, nbytes = qtype_geometry(qtype)
    b = _c(np.asarray(blocks_u8, dtype=np.uint8)).reshape(-1)
    nb = b.size // nbytes
    out = np.empty(nb * e, np.float32)
    lib().jo_dequant(int(qtype), _p(b), _p(out), nb)
    return out


def ref_dequant(qtype, blocks_u8):
    """Same through the reference's compiled src/quant.cpp (Q4_K and Q8_0 only:
    it has no CPU Q6_K routine)."""
    e, nbytes = qtype_geometry(qtype)
    b = _c(np.asarray(blocks_u8, dtype=np.uint8)).reshape(-1)
    nb = b.size // nbytes
    out = np.empty(nb * e, np.float32)
    fn = {Q4_K: "jref_dequantize_q4_K", Q8_0: "jref_dequantize_q8_0",
          Q4_0: "jref_dequantize_q4_0"}[qtype]
    getattr(ref(), fn)(_p(b), _p(out), nb)
    return out


def matvec(qtype, W_u8, x):
    """W uint8 [rows, cols/elems*bytes] of qtype, x fp32 [cols] -> (y fp32 [rows],
    sum_j |w_j x_j| fp64 [rows])."""
    e, nbytes = qtype_geometry(qtype)
    W = _c(np.asarray(W_u8, dtype=np.uint8))
    x = _c(np.asarray(x, dtype=np.float32))
    rows, cols = W.shape[0], x.shape[0]
    assert cols % e == 0 and W.shape[1] == cols // e * nbytes
    y = np.empty(rows, np.float32)
    a = np.empty(rows, np.float64)
    lib().jo_matvec(int(qtype), _p(W), _p(x), _p(y), _p(a), rows, cols)
    return y, a


# ---- GQA decode attention ----

def attention(q, k_cache, v_cache, lens, n_heads, n_heads_kv, head_dim, scale=None):
    """q fp32 [n_seq, n_heads*head_dim]; caches [n_seq, max_ctx, n_heads_kv*head_dim]
    (fp32 or fp16, same dtype); lens int32 [n_seq] (positions read per sequence).
    Returns (out fp32 [n_seq, n_heads*head_dim], sum_t p_t |v_t| fp64, same shape)."""
    q = _c(np.asarray(q, dtype=np.float32))
    k = _c(k_cache)
    v = _c(v_cache)
    assert k.dtype == v.dtype and k.shape == v.shape
    n_seq, max_ctx, kvw = k.shape
    assert kvw == n_heads_kv * head_dim and q.shape == (n_seq, n_heads * head_dim)
    lens = _c(np.asarray(lens, dtype=np.int32))
    assert head_dim <= 1024 and n_heads % n_heads_kv == 0
    if scale is None:
        scale = 1.0 / np.sqrt(float(head_dim))
    out = np.empty((n_seq, n_heads * head_dim), np.float32)
    a = np.empty((n_seq, n_heads * head_dim), np.float64)
    lib().jo_attention(_p(out), n_heads * head_dim, _p(q), n_heads * head_dim, _p(k), _p(v),
                       _act(k), kvw, max_ctx * kvw, _p(lens), n_seq, head_dim, n_heads,
                       n_heads_kv, float(scale), _p(a))
    return out, a
