"""Pins the oracle's decode loop (oracle/engine.py, the composition of the
per-kernel restatements along src/engine.cpp:684-805) against an independent
float64 textbook Llama decoder written from the mathematics: RMSNorm, RoPE as
a complex rotation z * e^{i pos theta_k}, GQA softmax attention over the
positions so far, SwiGLU, residual stream.  A dropped residual, a wrong
rotation pair or angle, a K/V row stored at the wrong position or a wrong
head grouping moves the logits by O(1); the fp32 stages of the composition
move them by about 1e-6 of their scale.  Also the greedy tie and NaN rules,
and the engine C-ABI's host-side argument checks (no GPU needed)."""
import ctypes

import numpy as np
import pytest

import jinf_amd
import model_util as mu
import oracle
from oracle import engine as oeng


def dense(W, name, hp):
    a, qt = W[name]
    if qt in (oracle.F32, oracle.F16):
        return np.asarray(a, np.float64)
    rows = a.shape[0]
    return oracle.dequant(qt, a).astype(np.float64).reshape(rows, -1)


def textbook_logits(hp, W, tokens):
    """float64 decode; returns the logits after every token."""
    n, nh, nkv = hp["n_embd"], hp["n_heads"], hp["n_heads_kv"]
    hd = n // nh
    eps, base = hp["rms_norm_eps"], hp["rope_freq_base"]
    M = {k: dense(W, k, hp) for k in W}
    theta = base ** (-np.arange(0, hd, 2, dtype=np.float64) / hd)

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + eps) * g

    def rot(vec, heads, pos):
        c = vec.reshape(heads, hd // 2, 2)
        z = (c[..., 0] + 1j * c[..., 1]) * np.exp(1j * pos * theta)
        return np.stack([z.real, z.imag], axis=-1).reshape(-1)

    K = [[] for _ in range(hp["n_layers"])]
    V = [[] for _ in range(hp["n_layers"])]
    E = dense(W, "token_embd.weight", hp).reshape(hp["n_vocab"], n)
    out_name = "output.weight" if "output.weight" in W else "token_embd.weight"
    logits = []
    for pos, tok in enumerate(tokens):
        h = E[tok].copy()
        for L in range(hp["n_layers"]):
            b = f"blk.{L}."
            x = rms(h, M[b + "attn_norm.weight"])
            q = rot(M[b + "attn_q.weight"] @ x, nh, pos)
            K[L].append(rot(M[b + "attn_k.weight"] @ x, nkv, pos))
            V[L].append(M[b + "attn_v.weight"] @ x)
            Ks, Vs = np.array(K[L]), np.array(V[L])
            o = np.empty(nh * hd)
            for hh in range(nh):
                j = hh // (nh // nkv)
                s = Ks[:, j * hd:(j + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                o[hh * hd:(hh + 1) * hd] = p @ Vs[:, j * hd:(j + 1) * hd]
            h = h + M[b + "attn_output.weight"] @ o
            x = rms(h, M[b + "ffn_norm.weight"])
            g = M[b + "ffn_gate.weight"] @ x
            u = M[b + "ffn_up.weight"] @ x
            h = h + M[b + "ffn_down.weight"] @ (g / (1.0 + np.exp(-g)) * u)
        if "output_norm.weight" in W:
            h = rms(h, M["output_norm.weight"])
        logits.append(M[out_name].reshape(hp["n_vocab"], n) @ h)
    return logits


def check_close(got, ref, what):
    scale = float(np.max(np.abs(ref)))
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    assert err <= 2e-5 * scale, f"{what}: {err:.3e} vs scale {scale:.3e}"


MODELS = {
    "mixed": dict(),
    "q4_0-f16-norms-tied": dict(types={k: mu.Q4_0 for k in mu.MIXED}, norm_type=mu.F16,
                                embd_type=mu.Q4_0, tied=True),
    "mha-hd128-q8": dict(n_embd=256, n_heads=2, n_heads_kv=2, types={k: mu.Q8_0 for k in mu.MIXED},
                         embd_type=mu.F16, out_type=mu.Q8_0),
    "no-output-norm-f32-embd": dict(n_layers=1, embd_type=mu.F32, output_norm=False),
    "gqa-8-to-1": dict(n_embd=512, n_heads=8, n_heads_kv=1, n_ff=256, n_layers=1),
}


@pytest.mark.parametrize("name", list(MODELS))
def test_composition_matches_textbook(name):
    hp, W = mu.tiny_model(seed=3, n_vocab=300, **MODELS[name])
    tokens = [5, 17, 299, 0, 42, 17]
    ref = textbook_logits(hp, W, tokens)
    dec = oeng.Decoder(hp, W, max_context=8)
    for t, (tok, r) in enumerate(zip(tokens, ref)):
        check_close(dec.step(tok), r, f"{name} token {t}")


def _planted(name, fn, hp, W, tokens):
    saved = getattr(oeng, name)
    setattr(oeng, name, fn(saved))
    try:
        dec = oeng.Decoder(hp, W, max_context=8)
        return [dec.step(t) for t in tokens]
    finally:
        setattr(oeng, name, saved)


def test_composition_detects_planted_mistakes():
    """Decoders with a planted mistake -- RoPE angles at twice the position
    (a uniform shift would cancel: attention sees only relative positions),
    or attention over n_past instead of n_past + 1 positions -- no longer
    match the textbook."""
    hp, W = mu.tiny_model(seed=4, n_vocab=200)
    tokens = [1, 2, 3, 4]
    ref = textbook_logits(hp, W, tokens)

    def doubled(rope):
        return lambda q, k, hd, positions=None, base=10000.0, **kw: rope(
            q, k, hd, positions=[2 * positions[0]], base=base)

    def short(att):
        return lambda q, kc, vc, lens, *a, **kw: att(q, kc, vc, [lens[0] - 1], *a, **kw)

    for name, fn in (("rope_rows", doubled), ("attention", short)):
        got = _planted(name, fn, hp, W, tokens)
        errs = [np.max(np.abs(g - r)) / np.max(np.abs(r)) for g, r in zip(got, ref)]
        assert max(errs) > 1e-2, name


def test_first_argmax_rules():
    assert oeng.first_argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert oeng.first_argmax(np.array([-0.0, 0.0, -1.0], np.float32)) == 0
    assert oeng.first_argmax(np.array([np.nan, 5.0, 1.0], np.float32)) == 0
    assert oeng.first_argmax(np.array([1.0, np.nan, 5.0, np.nan], np.float32)) == 2
    assert oeng.first_argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    x = np.random.default_rng(0).normal(size=1000).astype(np.float32)
    best, bv = 0, x[0]
    for j in range(1, x.size):     # the reference's scan, literally
        if x[j] > bv:
            best, bv = j, x[j]
    assert oeng.first_argmax(x) == best


def test_generate_stops_at_context_end():
    hp, W = mu.tiny_model(seed=5, n_vocab=64, n_layers=1)
    dec = oeng.Decoder(hp, W, max_context=6)
    out = dec.generate([1, 2, 3, 4], 10)
    assert dec.n_past == 6
    assert len(out) == 3 or out[-1] == oeng.EOS


# ---- the engine C-ABI on the host: argument checks before any HIP call ----

def _desc(**over):
    d = jinf_amd.engine.EngineDesc()
    vals = dict(n_layers=0, n_embd=256, n_heads=4, n_heads_kv=2, n_ff=512, n_vocab=100,
                max_context=16, rms_norm_eps=1e-5, rope_freq_base=1e4, kv_type=0,
                token_embd=0x1000, token_embd_type=mu.Q4_0, output=0x1000, output_type=mu.Q4_0)
    vals.update(over)
    for k, v in vals.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("over", [
    dict(n_embd=250),                       # n_embd % n_heads
    dict(n_heads_kv=3),                     # n_heads % n_heads_kv
    dict(n_embd=4 * 1026, n_heads=4),       # head_dim > 512
    dict(n_embd=12, n_heads=4),             # odd head_dim
    dict(kv_type=7),
    dict(max_context=0),
    dict(n_vocab=0),
    dict(token_embd=None),
    dict(token_embd_type=3),                # Q4_1: not served
    dict(output_type=mu.Q4_K, n_embd=288, n_heads=4),   # 288 not whole Q4_K blocks
    dict(output=None, token_embd_type=mu.F32),           # tied output needs a block type
    dict(n_layers=1),                       # no layer array
    dict(rope_freq_base=0.0),
])
def test_create_rejects_bad_descriptions(over):
    h = ctypes.c_void_p(0x1234)
    d = _desc(**over)
    assert jinf_amd.lib().jinf_hip_engine_create(ctypes.byref(h), ctypes.byref(d)) == 5
    assert h.value is None


def test_create_rejects_missing_layer_weights():
    layers = (jinf_amd.engine.LayerWeights * 1)()
    for n in mu.LAYER_TENSORS:
        setattr(layers[0], n, 0x1000)
        setattr(layers[0], n + "_type", mu.F32 if n.endswith("norm") else mu.Q4_0)
    layers[0].ffn_down = None
    d = _desc(n_layers=1)
    d.layers = layers
    h = ctypes.c_void_p()
    assert jinf_amd.lib().jinf_hip_engine_create(ctypes.byref(h), ctypes.byref(d)) == 5
    layers[0].ffn_down = 0x1000
    layers[0].attn_q_type = mu.F32          # a dense matrix: not served
    assert jinf_amd.lib().jinf_hip_engine_create(ctypes.byref(h), ctypes.byref(d)) == 5


def test_null_arguments():
    L = jinf_amd.lib()
    h = ctypes.c_void_p()
    n = ctypes.c_int(0)
    p = ctypes.c_void_p()
    assert L.jinf_hip_engine_create(None, None) == 5
    assert L.jinf_hip_engine_create(ctypes.byref(h), None) == 5
    assert L.jinf_hip_engine_create_gguf(ctypes.byref(h), None, 16, 0, 0) == 5
    assert L.jinf_hip_engine_forward(None, None, 1, ctypes.byref(p)) == 5
    assert L.jinf_hip_engine_generate(None, None, 0, None, 4, ctypes.byref(n)) == 5
    assert L.jinf_hip_engine_reset(None) == 5
    assert L.jinf_hip_engine_n_past(None) == -1
    assert L.jinf_hip_engine_use_graph(None, 1) == 5
    assert L.jinf_hip_engine_copy_logits(None, None, 0) == 5
    assert L.jinf_hip_engine_step_weight_bytes(None) == 0
    L.jinf_hip_engine_destroy(None)
