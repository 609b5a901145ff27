"""CPU restatement of jinf's per-token decode loop, composed from the oracle's
per-kernel functions.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the GPU decode
engine; the product path never imports it.

Follows src/engine.cpp: embedding (:311-334), per layer (:418-511) RMSNorm,
Q/K/V GEMVs, RoPE at position n_past, K/V rows into the cache at n_past,
attention over n_past + 1 positions, output GEMV, residual add, FFN RMSNorm,
gate/up GEMVs, SiLU * up, down GEMV, residual add; then the final RMSNorm and
the output GEMV (:736-747), and greedy generation (:762-805).  Every stage
stores fp32 like the reference's buffers; each kernel is the oracle's
restatement (each pinned on its own), and the composition itself is pinned
against an independent float64 textbook decoder in
tests/test_oracle_engine.py.

Weights: {GGUF tensor name: (numpy array, jinf_qtype code)}; a block type is
uint8 [rows, row bytes], F32 / F16 a float32 / float16 array.
"""
import numpy as np

from . import (F16, F32, attention, dequant, matvec, qtype_geometry, residual_add,
               residual_rmsnorm_rows, rmsnorm_rows, rope_rows, swiglu)

LAYER_TENSORS = ("attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                 "ffn_gate", "ffn_up", "ffn_down")
EOS = 2


def embed_row(table, qtype, tok, n_embd):
    """Dequantized embedding row `tok` (src/engine.cpp:311-334; the F16 table,
    which the reference leaves unhandled, is widened exactly)."""
    if qtype == F32:
        return np.asarray(table, np.float32).reshape(-1, n_embd)[tok].copy()
    if qtype == F16:
        return np.asarray(table, np.float16).reshape(-1, n_embd)[tok].astype(np.float32)
    e, b = qtype_geometry(qtype)
    return dequant(qtype, np.asarray(table, np.uint8).reshape(-1, n_embd // e * b)[tok])


def first_argmax(x):
    """The reference's greedy pick (src/engine.cpp:783-791): scan from element
    0, keep strict improvements -> first index of the largest value; NaNs
    after element 0 are skipped, a NaN element 0 is never improved on."""
    x = np.asarray(x, np.float32)
    if np.isnan(x[0]):
        return 0
    m = np.nanmax(x)
    return int(np.flatnonzero(x == m)[0])


class Decoder:
    """State of one decode (KV caches, n_past) over a model's weights."""

    def __init__(self, hp, weights, max_context, kv_type=F32):
        self.hp = hp
        self.w = weights
        self.max_context = max_context
        self.n_embd = hp["n_embd"]
        self.hd = hp["n_embd"] // hp["n_heads"]
        self.kvd = hp["n_heads_kv"] * self.hd
        self.eps = float(np.float32(hp.get("rms_norm_eps", 1e-5)))
        self.base = float(np.float32(hp.get("rope_freq_base", 10000.0)))
        dt = np.float16 if kv_type == F16 else np.float32
        self.kc = [np.zeros((1, max_context, self.kvd), dt) for _ in range(hp["n_layers"])]
        self.vc = [np.zeros((1, max_context, self.kvd), dt) for _ in range(hp["n_layers"])]
        self.n_past = 0
        self.last_logits = None

    def _mv(self, name, x):
        W, qt = self.w[name]
        return matvec(qt, W, x)[0]

    def _norm_w(self, name):
        return self.w[name][0]

    def step(self, tok):
        """One token at position n_past; returns its fp32 logits."""
        hp, n, hd, pos = self.hp, self.n_embd, self.hd, self.n_past
        assert pos < self.max_context
        tab, tq = self.w["token_embd.weight"]
        hidden = embed_row(tab, tq, tok, n)[None]
        delta = None
        for L in range(hp["n_layers"]):
            b = f"blk.{L}."
            if delta is None:
                x = rmsnorm_rows(hidden, self._norm_w(b + "attn_norm.weight"), self.eps)
            else:
                hidden, x = residual_rmsnorm_rows(hidden, delta,
                                                  self._norm_w(b + "attn_norm.weight"), self.eps)
            q = self._mv(b + "attn_q.weight", x[0])
            k = self._mv(b + "attn_k.weight", x[0])
            v = self._mv(b + "attn_v.weight", x[0])
            q, k = rope_rows(q[None], k[None], hd, positions=[pos], base=self.base)
            self.kc[L][0, pos] = k[0].astype(self.kc[L].dtype)
            self.vc[L][0, pos] = v.astype(self.vc[L].dtype)
            att, _ = attention(q, self.kc[L], self.vc[L], [pos + 1], hp["n_heads"],
                               hp["n_heads_kv"], hd)
            proj = self._mv(b + "attn_output.weight", att[0])
            hidden, x = residual_rmsnorm_rows(hidden, proj[None],
                                              self._norm_w(b + "ffn_norm.weight"), self.eps)
            g = self._mv(b + "ffn_gate.weight", x[0])
            u = self._mv(b + "ffn_up.weight", x[0])
            delta = self._mv(b + "ffn_down.weight", swiglu(g, u))[None]
        if "output_norm.weight" in self.w:
            onw = self._norm_w("output_norm.weight")
            if delta is None:
                x = rmsnorm_rows(hidden, onw, self.eps)
            else:
                hidden, x = residual_rmsnorm_rows(hidden, delta, onw, self.eps)
        else:
            x = hidden if delta is None else residual_add(hidden, delta)
        out = "output.weight" if "output.weight" in self.w else "token_embd.weight"
        logits = self._mv(out, x[0])
        self.n_past += 1
        self.last_logits = logits
        return logits

    def forward(self, tokens):
        """jinf_engine_forward: every token in turn; the last token's logits."""
        for t in tokens:
            self.step(int(t))
        return self.last_logits

    def generate(self, prompt, max_tokens):
        """jinf_engine_generate (greedy, EOS id 2), stopping when the context
        is full as the reference does when its forward call fails."""
        if len(prompt):
            self.forward(prompt)
        assert self.n_past > 0
        out = []
        for _ in range(max_tokens):
            best = first_argmax(self.last_logits)
            out.append(best)
            if best == EOS or self.n_past >= self.max_context:
                break
            self.step(best)
        return out
