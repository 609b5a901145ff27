"""Torch-tensor front end over the jinf C-ABI (libjinf_hip.so).

Tensors must live on the current HIP device; every call is enqueued on torch's
current stream, and nothing synchronizes.  Shapes follow the reference engine:
rows are tokens (or (sequence, head) pairs for softmax), the last dimension is
contiguous, and the row stride is passed as the C-ABI `ld_*` argument.

Each function raises JinfError when the library rejects its arguments; there
is no CPU or PyTorch fallback.
"""
import ctypes

import torch

from ._lib import F16, F32, JINF_HIP_OK, Q4_0, Q4_K, Q6_K, Q8_0, lib


class JinfError(RuntimeError):
    pass


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _act(t):
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float16:
        return F16
    raise JinfError(f"unsupported dtype {t.dtype}")


def _rows(t):
    """(n_rows, n, ld) of a tensor viewed as rows over its last dimension."""
    if t.dim() == 1:
        return 1, t.shape[0], t.shape[0]
    if t.stride(-1) != 1:
        raise JinfError("last dimension must be contiguous")
    n = t.shape[-1]
    lead = t.shape[:-1]
    rows = 1
    for s in lead:
        rows *= s
    # leading dims must collapse onto one row stride
    ld = t.stride(-2)
    expect = ld
    for d in range(t.dim() - 2, -1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            raise JinfError("leading dimensions must form a single row stride")
        expect *= t.shape[d]
    return rows, n, ld


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _check(rc, name):
    if rc != JINF_HIP_OK:
        raise JinfError(f"{name} returned status {rc}")


def rmsnorm_rows(x, weight, eps=1e-5, out=None):
    """out[r] = rmsnorm(x[r]) * weight (x fp32 or fp16; weight fp32 or fp16)."""
    out = torch.empty_like(x) if out is None else out
    rows, n, ld_in = _rows(x)
    _, _, ld_out = _rows(out)
    _check(lib().jinf_rmsnorm_rows(_ptr(out), ld_out, _ptr(x), ld_in, _ptr(weight), rows, n,
                                   float(eps), _act(x), _act(weight), _stream()),
           "jinf_rmsnorm_rows")
    return out


def residual_rmsnorm_rows(residual, delta, weight, eps=1e-5, out=None):
    """residual += delta (in place, rounded to its dtype); returns rmsnorm(residual)*w."""
    out = torch.empty_like(residual) if out is None else out
    rows, n, ld_res = _rows(residual)
    _, _, ld_d = _rows(delta)
    _, _, ld_out = _rows(out)
    _check(lib().jinf_residual_rmsnorm_rows(_ptr(out), ld_out, _ptr(residual), ld_res,
                                            _ptr(delta), ld_d, _ptr(weight), rows, n,
                                            float(eps), _act(residual), _act(weight),
                                            _stream()),
           "jinf_residual_rmsnorm_rows")
    return out


def rope_rows(q, k, head_dim, positions=None, pos0=0, freq_base=10000.0):
    """In-place interleaved RoPE.  q: [T, n_heads*head_dim] (or [T, n_heads,
    head_dim]), k: [T, n_heads_kv*head_dim]; positions: int32 [T] or None."""
    T = q.shape[0]
    q2 = q.reshape(T, -1) if q.is_contiguous() else q
    k2 = k.reshape(T, -1) if k.is_contiguous() else k
    nh = q2.shape[1] // head_dim
    nkv = k2.shape[1] // head_dim
    if positions is not None and positions.dtype != torch.int32:
        raise JinfError("positions must be int32")
    _check(lib().jinf_rope_rows(_ptr(q2), q2.stride(0), _ptr(k2), k2.stride(0),
                                _ptr(positions), int(pos0), T, head_dim, nh, nkv,
                                float(freq_base), _act(q), _stream()),
           "jinf_rope_rows")
    return q, k


def swiglu(gate, up, out=None):
    """out = silu(gate) * up (out may be gate or up)."""
    out = torch.empty_like(gate) if out is None else out
    rows, n, ld_g = _rows(gate)
    _, _, ld_u = _rows(up)
    _, _, ld_o = _rows(out)
    _check(lib().jinf_swiglu_rows(_ptr(out), ld_o, _ptr(gate), ld_g, _ptr(up), ld_u, rows, n,
                                  _act(gate), _stream()),
           "jinf_swiglu_rows")
    return out


def residual_add(a, b):
    """a += b in place."""
    rows, n, ld_a = _rows(a)
    _, _, ld_b = _rows(b)
    _check(lib().jinf_residual_add_rows(_ptr(a), ld_a, _ptr(b), ld_b, rows, n, _act(a),
                                        _stream()),
           "jinf_residual_add_rows")
    return a


def softmax_rows(x, lens=None, rows_per_len=1, scale=1.0, out=None):
    """Masked fp32 row softmax; rows j >= len are left untouched in `out`."""
    out = torch.empty_like(x) if out is None else out
    rows, n, ld_in = _rows(x)
    _, _, ld_out = _rows(out)
    if lens is not None and lens.dtype != torch.int32:
        raise JinfError("lens must be int32")
    _check(lib().jinf_softmax_rows_f32(_ptr(out), ld_out, _ptr(x), ld_in, rows, n, _ptr(lens),
                                       int(rows_per_len), float(scale), _stream()),
           "jinf_softmax_rows_f32")
    return out


def embed_q4_0(table, ids, n_embd, out_dtype=torch.float16, out=None):
    """Gather + dequantize rows of a Q4_0 table (uint8 [n_vocab, n_embd/32*18])."""
    n_vocab = table.shape[0]
    n_ids = ids.shape[0] if ids is not None else n_vocab
    if out is None:
        out = torch.empty((n_ids, n_embd), dtype=out_dtype, device=table.device)
    if ids is not None and ids.dtype != torch.int32:
        raise JinfError("ids must be int32")
    _check(lib().jinf_embed_q4_0(_ptr(out), out.stride(0), _ptr(table), n_vocab, n_embd,
                                 _ptr(ids), n_ids, _act(out), _stream()),
           "jinf_embed_q4_0")
    return out


_GEOM = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def matvec_q4_0(weight, x, y=None):
    """y = W x: weight uint8 [rows, cols/32*18] (Q4_0 blocks), x fp32 [cols]."""
    return matvec(weight, x, Q4_0, y)


def matvec(weight, x, qtype, y=None):
    """y = W x: weight uint8 [rows, cols/elems*bytes] of qtype blocks, x fp32 [cols]."""
    if qtype not in _GEOM:
        raise JinfError(f"unsupported qtype {qtype}")
    elems, nbytes = _GEOM[qtype]
    rows = weight.shape[0]
    cols = x.shape[0]
    if weight.shape[1] != cols // elems * nbytes:
        raise JinfError("weight row bytes do not match cols")
    y = torch.empty(rows, dtype=torch.float32, device=x.device) if y is None else y
    _check(lib().jinf_matvec(_ptr(weight), int(qtype), _ptr(x), _ptr(y), rows, cols, _stream()),
           "jinf_matvec")
    return y


def _mv_shape(weight, qtype, cols):
    if qtype not in _GEOM:
        raise JinfError(f"unsupported qtype {qtype}")
    elems, nbytes = _GEOM[qtype]
    if weight.shape[1] != cols // elems * nbytes:
        raise JinfError("weight row bytes do not match cols")
    return weight.shape[0]


def _norm_args(norm_w):
    if norm_w is None:
        return None, F32
    return _ptr(norm_w), (F16 if norm_w.dtype == torch.float16 else F32)


def rmsnorm_matvec(weight, h, qtype, norm_w=None, eps=1e-5, y=None):
    """y = W (rmsnorm(h) * g) in one launch (norm_w None: y = W h)."""
    rows = _mv_shape(weight, qtype, h.shape[0])
    y = torch.empty(rows, dtype=torch.float32, device=h.device) if y is None else y
    nw, nt = _norm_args(norm_w)
    _check(lib().jinf_rmsnorm_matvec(_ptr(weight), int(qtype), _ptr(h), nw, nt, float(eps),
                                     _ptr(y), rows, h.shape[0], _stream()),
           "jinf_rmsnorm_matvec")
    return y


def matvec_add(weight, x, qtype, y):
    """y += W x in place (the residual add fused into the GEMV)."""
    rows = _mv_shape(weight, qtype, x.shape[0])
    _check(lib().jinf_matvec_add(_ptr(weight), int(qtype), _ptr(x), _ptr(y), rows, x.shape[0],
                                 _stream()), "jinf_matvec_add")
    return y


def rmsnorm_swiglu_matvec(w_gate, w_up, h, qtype, norm_w=None, eps=1e-5, out=None):
    """out = silu(W_gate x^) * (W_up x^), x^ = rmsnorm(h) * g, one launch."""
    n_ff = _mv_shape(w_gate, qtype, h.shape[0])
    if tuple(w_up.shape) != tuple(w_gate.shape):
        raise JinfError("gate and up shapes differ")
    out = torch.empty(n_ff, dtype=torch.float32, device=h.device) if out is None else out
    nw, nt = _norm_args(norm_w)
    _check(lib().jinf_rmsnorm_swiglu_matvec(_ptr(w_gate), _ptr(w_up), int(qtype), _ptr(h), nw,
                                            nt, float(eps), _ptr(out), n_ff, h.shape[0],
                                            _stream()), "jinf_rmsnorm_swiglu_matvec")
    return out


def rmsnorm_qkv_rope(w_q, w_k, w_v, h, qtype, pos, k_cache, v_cache, head_dim, n_heads,
                     n_heads_kv, freq_base, norm_w=None, eps=1e-5, q_out=None):
    """q = rope(W_q x^) (returned); rope(W_k x^) and W_v x^ stored into the
    cache rows at device position pos[0] (caches [max_ctx, n_heads_kv *
    head_dim], fp32 or fp16).  A None weight skips its projection."""
    cols = h.shape[0]
    for w in (w_q, w_k, w_v):
        if w is not None:
            _mv_shape(w, qtype, cols)
    if w_q is not None and q_out is None:
        q_out = torch.empty(n_heads * head_dim, dtype=torch.float32, device=h.device)
    cache = k_cache if k_cache is not None else v_cache
    kv_type = _act(cache) if cache is not None else F32
    max_ctx = cache.shape[0] if cache is not None else 0
    nw, nt = _norm_args(norm_w)
    _check(lib().jinf_rmsnorm_qkv_rope(_ptr(w_q), _ptr(w_k), _ptr(w_v), int(qtype), _ptr(h), nw,
                                       nt, float(eps), cols, _ptr(q_out), _ptr(k_cache),
                                       _ptr(v_cache), kv_type, _ptr(pos), max_ctx, head_dim,
                                       n_heads, n_heads_kv, float(freq_base), _stream()),
           "jinf_rmsnorm_qkv_rope")
    return q_out


def matvec_batch_workspace(rows, cols, n_batch, device="cuda"):
    """A zero-filled workspace tensor for the batched GEMVs (prepared x, and
    the split partials and counters; counters must start at zero, calls
    leave them so)."""
    nbytes = lib().jinf_matvec_batch_workspace_bytes(rows, cols, n_batch)
    return torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)


def _ws(workspace, rows, cols, n_batch, device):
    if workspace is None:
        workspace = matvec_batch_workspace(rows, cols, n_batch, device)
    return _ptr(workspace), workspace.numel()


def _mb_rows(weight, qtype, x):
    if x.dim() != 2 or x.dtype != torch.float32:
        raise JinfError("x must be fp32 [n_batch, cols]")
    return _mv_shape(weight, qtype, x.shape[1])


def matvec_batch(weight, x, qtype, y=None, workspace=None):
    """y[b] = W x[b] on the matrix cores; x fp32 [n_batch, cols]."""
    rows = _mb_rows(weight, qtype, x)
    n_batch, cols = x.shape
    y = torch.empty((n_batch, rows), dtype=torch.float32, device=x.device) if y is None else y
    wp, wn = _ws(workspace, rows, cols, n_batch, x.device)
    _check(lib().jinf_matvec_batch(_ptr(weight), int(qtype), _ptr(x), x.stride(0), _ptr(y),
                                   y.stride(0), rows, cols, n_batch, wp, wn, _stream()),
           "jinf_matvec_batch")
    return y


def matvec_batch_add(weight, x, qtype, y, workspace=None):
    """y[b] += W x[b] in place."""
    rows = _mb_rows(weight, qtype, x)
    n_batch, cols = x.shape
    wp, wn = _ws(workspace, rows, cols, n_batch, x.device)
    _check(lib().jinf_matvec_batch_add(_ptr(weight), int(qtype), _ptr(x), x.stride(0), _ptr(y),
                                       y.stride(0), rows, cols, n_batch, wp, wn, _stream()),
           "jinf_matvec_batch_add")
    return y


def rmsnorm_matvec_batch(weight, h, qtype, norm_w, eps=1e-5, y=None, workspace=None):
    """y[b] = W (rmsnorm(h[b]) * g)."""
    rows = _mb_rows(weight, qtype, h)
    n_batch, cols = h.shape
    y = torch.empty((n_batch, rows), dtype=torch.float32, device=h.device) if y is None else y
    nw, nt = _norm_args(norm_w)
    wp, wn = _ws(workspace, rows, cols, n_batch, h.device)
    _check(lib().jinf_rmsnorm_matvec_batch(_ptr(weight), int(qtype), _ptr(h), h.stride(0), nw,
                                           nt, float(eps), _ptr(y), y.stride(0), rows, cols,
                                           n_batch, wp, wn, _stream()),
           "jinf_rmsnorm_matvec_batch")
    return y


def rmsnorm_swiglu_matvec_batch(w_gate, w_up, h, qtype, norm_w, eps=1e-5, out=None,
                                workspace=None):
    """out[b] = silu(W_gate x^[b]) * (W_up x^[b])."""
    n_ff = _mb_rows(w_gate, qtype, h)
    if tuple(w_up.shape) != tuple(w_gate.shape):
        raise JinfError("gate and up shapes differ")
    n_batch, cols = h.shape
    out = torch.empty((n_batch, n_ff), dtype=torch.float32, device=h.device) if out is None else out
    nw, nt = _norm_args(norm_w)
    wp, wn = _ws(workspace, n_ff, cols, n_batch, h.device)
    _check(lib().jinf_rmsnorm_swiglu_matvec_batch(_ptr(w_gate), _ptr(w_up), int(qtype), _ptr(h),
                                                  h.stride(0), nw, nt, float(eps), _ptr(out),
                                                  out.stride(0), n_ff, cols, n_batch, wp, wn,
                                                  _stream()),
           "jinf_rmsnorm_swiglu_matvec_batch")
    return out


def rmsnorm_qkv_rope_batch(w_q, w_k, w_v, h, qtype, norm_w, positions, k_cache, v_cache,
                           head_dim, n_heads, n_heads_kv, freq_base, eps=1e-5, q_out=None,
                           workspace=None):
    """Per sequence b: q[b] = rope(W_q x^[b]) (returned); rope(W_k x^[b]) and
    W_v x^[b] stored at positions[b] of k_cache / v_cache [n_batch, max_ctx,
    n_heads_kv * head_dim] (fp32 or fp16)."""
    n_batch, cols = h.shape
    rows = 0
    for w in (w_q, w_k, w_v):
        if w is not None:
            rows += _mv_shape(w, qtype, cols)
    if w_q is not None and q_out is None:
        q_out = torch.empty((n_batch, n_heads * head_dim), dtype=torch.float32, device=h.device)
    cache = k_cache if k_cache is not None else v_cache
    kv_type = _act(cache) if cache is not None else F32
    max_ctx = cache.shape[1] if cache is not None else 0
    ld_seq = cache.stride(0) if cache is not None else 0
    nw, nt = _norm_args(norm_w)
    wp, wn = _ws(workspace, max(rows, 1), cols, n_batch, h.device)
    _check(lib().jinf_rmsnorm_qkv_rope_batch(
        _ptr(w_q), _ptr(w_k), _ptr(w_v), int(qtype), _ptr(h), h.stride(0), nw, nt, float(eps),
        cols, _ptr(q_out), q_out.stride(0) if q_out is not None else 0, _ptr(k_cache),
        _ptr(v_cache), kv_type, ld_seq, _ptr(positions), max_ctx, head_dim, n_heads, n_heads_kv,
        float(freq_base), n_batch, wp, wn, _stream()), "jinf_rmsnorm_qkv_rope_batch")
    return q_out


def dequant_rows(table, qtype, n_embd, ids=None, out_dtype=torch.float32, out=None):
    """Gather + dequantize rows of a qtype table (uint8 [n_vocab, row bytes])."""
    n_vocab = table.shape[0]
    n_ids = ids.shape[0] if ids is not None else n_vocab
    if out is None:
        out = torch.empty((n_ids, n_embd), dtype=out_dtype, device=table.device)
    if ids is not None and ids.dtype != torch.int32:
        raise JinfError("ids must be int32")
    _check(lib().jinf_dequant_rows(_ptr(out), out.stride(0), _ptr(table), int(qtype), n_vocab,
                                   n_embd, _ptr(ids), n_ids, _act(out), _stream()),
           "jinf_dequant_rows")
    return out


def attention_workspace(n_seq, n_heads, head_dim, max_ctx, device="cuda"):
    """A zero-filled workspace tensor for attention_decode's split of long
    contexts (its merge counters must start at zero; calls leave them so)."""
    nbytes = lib().jinf_attention_workspace_bytes(n_seq, n_heads, head_dim, max_ctx)
    return torch.zeros(max(nbytes, 4), dtype=torch.uint8, device=device)


def attention_decode(q, k_cache, v_cache, lens, n_heads, n_heads_kv, scale=0.0, out=None,
                     workspace=None):
    """Batched GQA decode attention.  q fp32 [n_seq, n_heads*hd]; caches
    [n_seq, max_ctx, n_heads_kv*hd] fp32 or fp16 (same dtype); lens int32
    [n_seq]; workspace: optional uint8 tensor (attention_workspace).  Returns
    out fp32 [n_seq, n_heads*hd]."""
    n_seq, max_ctx, kvw = k_cache.shape
    hd = kvw // n_heads_kv
    if v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise JinfError("k and v caches must match")
    if lens.dtype != torch.int32:
        raise JinfError("lens must be int32")
    out = torch.empty((n_seq, n_heads * hd), dtype=torch.float32, device=q.device) if out is None else out
    _check(lib().jinf_attention_decode(_ptr(out), out.stride(0), _ptr(q), q.stride(0),
                                       _ptr(k_cache), _ptr(v_cache), _act(k_cache),
                                       k_cache.stride(1), k_cache.stride(0), _ptr(lens), n_seq,
                                       max_ctx, hd, n_heads, n_heads_kv, float(scale),
                                       _ptr(workspace),
                                       0 if workspace is None else workspace.numel(), _stream()),
           "jinf_attention_decode")
    return out


# ---- drop-in entry points (reference signatures; fp32, one row) ----

def cuda_rmsnorm(out, x, weight, eps=1e-5):
    wt = F16 if weight.dtype == torch.float16 else F32
    lib().jinf_cuda_rmsnorm(_ptr(out), _ptr(x), _ptr(weight), x.numel(), float(eps), wt,
                            _stream())
    return out


def cuda_rope(q, k, head_dim, n_heads, n_heads_kv, pos, freq_base):
    lib().jinf_cuda_rope(_ptr(q), _ptr(k), head_dim, n_heads, n_heads_kv, int(pos),
                         float(freq_base), _stream())
    return q, k


def cuda_silu_mul(out, gate, up):
    lib().jinf_cuda_silu_mul(_ptr(out), _ptr(gate), _ptr(up), gate.numel(), _stream())
    return out


def cuda_softmax(out, x):
    lib().jinf_cuda_softmax(_ptr(out), _ptr(x), x.numel(), _stream())
    return out


def cuda_residual_add(a, b):
    lib().jinf_cuda_residual_add(_ptr(a), _ptr(b), a.numel(), _stream())
    return a


def cuda_dequant_matvec(weight, x, y, rows, cols, qtype=2):
    lib().jinf_cuda_dequant_matvec(_ptr(weight), _ptr(x), _ptr(y), int(rows), int(cols),
                                   int(qtype), _stream())
    return y


def cuda_dequantize_q4_0(data, out, n_blocks, byte_offset=0):
    ptr = ctypes.c_void_p(data.data_ptr() + byte_offset)
    lib().jinf_cuda_dequantize_q4_0(ptr, _ptr(out), int(n_blocks), _stream())
    return out


def cuda_dequantize(qtype, data, out, n_blocks, byte_offset=0):
    """The reference's per-row launchers jinf_cuda_dequantize_{q4_0,q8_0,q4_K,q6_K}."""
    name = {Q4_0: "jinf_cuda_dequantize_q4_0", Q8_0: "jinf_cuda_dequantize_q8_0",
            Q4_K: "jinf_cuda_dequantize_q4_K", Q6_K: "jinf_cuda_dequantize_q6_K"}[qtype]
    ptr = ctypes.c_void_p(data.data_ptr() + byte_offset)
    getattr(lib(), name)(ptr, _ptr(out), int(n_blocks), _stream())
    return out


def cuda_attention(out, q, k_cache, v_cache, head_dim, n_heads, n_heads_kv, n_past, max_ctx):
    lib().jinf_cuda_attention(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), int(head_dim),
                              int(n_heads), int(n_heads_kv), int(n_past), int(max_ctx), _stream())
    return out


# ---- bandwidth probes (include/jinf/probe_hip.h): bench.py's ceilings ----

def probe_rows_inplace(a, b, units_per_lane=1, exchange=True):
    """RoPE's traffic, in place: rows of a [T, *] and b [T, *] (same T), every
    live byte read and rewritten (the data becomes meaningless)."""
    ra, na, lda = _rows(a)
    rb, nb, ldb = _rows(b)
    es = a.element_size()
    _check(lib().jinf_probe_rows_inplace(_ptr(a), lda * es, na * es // 16, _ptr(b),
                                         ldb * b.element_size(), nb * b.element_size() // 16,
                                         ra, int(units_per_lane), int(bool(exchange)),
                                         _stream()), "jinf_probe_rows_inplace")


def probe_stream(out0, in0, out1=None, in1=None, units_per_lane=1, exchange=True):
    """Flat streams of out0.numel() * element_size bytes (16-byte units)."""
    nbytes = out0.numel() * out0.element_size()
    _check(lib().jinf_probe_stream(_ptr(out0), _ptr(out1), _ptr(in0), _ptr(in1), nbytes // 16,
                                   int(units_per_lane), int(bool(exchange)), _stream()),
           "jinf_probe_stream")


def probe_stream_layout(out0, in0, out1=None, in1=None, units_per_lane=1, exchange=True,
                        block_lanes=256, max_groups=0):
    """probe_stream in a chosen launch layout: block_lanes lanes per workgroup,
    one pass (max_groups 0) or a grid-stride loop over max_groups workgroups;
    exchange False / True, or 2: out0 stored straight after its own loads,
    out1 after the cross-lane exchange."""
    nbytes = out0.numel() * out0.element_size()
    _check(lib().jinf_probe_stream_layout(_ptr(out0), _ptr(out1), _ptr(in0), _ptr(in1),
                                          nbytes // 16, int(units_per_lane), int(exchange),
                                          int(block_lanes), int(max_groups), _stream()),
           "jinf_probe_stream_layout")


def probe_read_layout(inp, sink, units_per_lane=1, block_lanes=256, max_groups=0):
    """A read-only stream over inp's bytes (16-byte units) in a chosen launch
    layout; sink: a 4-byte device tensor the probe leaves untouched in practice."""
    nbytes = inp.numel() * inp.element_size()
    _check(lib().jinf_probe_read_layout(_ptr(inp), nbytes // 16, _ptr(sink), int(units_per_lane),
                                        int(block_lanes), int(max_groups), _stream()),
           "jinf_probe_read_layout")


def probe_gather(out, table, ids, in_row_bytes, units_per_lane=1, exchange=True):
    """The gather's traffic: out row r from table row ids[r] (table viewed as
    byte rows; in_row_bytes of each row read)."""
    n_ids, n_out, ld_out = _rows(out)
    es = out.element_size()
    rows, _, ld_t = _rows(table)
    _check(lib().jinf_probe_gather(_ptr(out), ld_out * es, n_out * es // 16, _ptr(table),
                                   ld_t * table.element_size(), in_row_bytes // 16, rows,
                                   _ptr(ids), n_ids, int(units_per_lane), int(bool(exchange)),
                                   _stream()), "jinf_probe_gather")


def probe_rows_ragged(out, x, lens, rows_per_len):
    """The masked softmax's traffic over fp32 rows of x with lengths lens."""
    rows, n, ld_in = _rows(x)
    _, _, ld_out = _rows(out)
    _check(lib().jinf_probe_rows_ragged(_ptr(out), ld_out * 4, _ptr(x), ld_in * 4, n, _ptr(lens),
                                        int(rows_per_len), rows, _stream()),
           "jinf_probe_rows_ragged")
