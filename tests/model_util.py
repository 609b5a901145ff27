"""Tiny random Llama-style models for the decode-engine tests: weights named as
in GGUF files, as numpy arrays (the oracle's side) or device tensors (the
engine's side), and a GGUF writer for them."""
import numpy as np

import gguf_writer as gw
import oracle
import testutil as tu

F32, F16 = oracle.F32, oracle.F16
Q4_0, Q8_0, Q4_K, Q6_K = oracle.Q4_0, oracle.Q8_0, oracle.Q4_K, oracle.Q6_K
LAYER_TENSORS = ("attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                 "ffn_gate", "ffn_up", "ffn_down")

# per-layer matrix types, alternating between even and odd layers
MIXED = {"attn_q": (Q4_0, Q4_K), "attn_k": (Q8_0, Q6_K), "attn_v": (Q4_K, Q4_0),
         "attn_output": (Q6_K, Q8_0), "ffn_gate": (Q4_K, Q4_0), "ffn_up": (Q4_0, Q8_0),
         "ffn_down": (Q6_K, Q4_K)}


def matrix(seed, qt, rows, cols, rms=None):
    """Random [rows, cols] weight of type qt whose dequantized values have
    root-mean-square `rms` (default 1/sqrt(cols), so y = W x keeps the scale
    of x).  Dense types return float arrays."""
    rms = 1.0 / np.sqrt(cols) if rms is None else rms
    if qt in (F32, F16):
        w = tu.rng(seed).normal(0.0, rms, size=(rows, cols))
        return w.astype(np.float32 if qt == F32 else np.float16)
    probe = tu.quant_table(tu.rng(seed), qt, rows, cols, 0.01)
    got = float(np.sqrt(np.mean(oracle.dequant(qt, probe).astype(np.float64) ** 2)))
    return tu.quant_table(tu.rng(seed), qt, rows, cols, 0.01 * rms / got)


def norm_weight(seed, n, dtype):
    w = tu.rng(seed).normal(1.0, 0.1, size=n)
    return w.astype(np.float32 if dtype == F32 else np.float16)


def tiny_model(seed=0, n_layers=2, n_embd=256, n_heads=4, n_heads_kv=2, n_ff=512, n_vocab=1000,
               types=MIXED, norm_type=F32, embd_type=Q4_K, out_type=Q6_K, output_norm=True,
               tied=False, rope_freq_base=10000.0, eps=1e-5):
    """(hparams, {name: (array, qtype)}).  types: {tensor: qtype or
    (even-layer qtype, odd-layer qtype)}."""
    hd = n_embd // n_heads
    kvd = n_heads_kv * hd
    hp = dict(n_layers=n_layers, n_embd=n_embd, n_heads=n_heads, n_heads_kv=n_heads_kv,
              n_ff=n_ff, n_vocab=n_vocab, rope_freq_base=rope_freq_base, rms_norm_eps=eps)
    shapes = {"attn_q": (n_embd, n_embd), "attn_k": (kvd, n_embd), "attn_v": (kvd, n_embd),
              "attn_output": (n_embd, n_embd), "ffn_gate": (n_ff, n_embd),
              "ffn_up": (n_ff, n_embd), "ffn_down": (n_embd, n_ff)}
    W = {}
    s = seed * 1000
    W["token_embd.weight"] = (matrix(s + 1, embd_type, n_vocab, n_embd, rms=1.0), embd_type)
    for L in range(n_layers):
        for i, name in enumerate(LAYER_TENSORS):
            key = f"blk.{L}.{name}.weight"
            sd = s + 10 + 20 * L + i
            if name.endswith("norm"):
                W[key] = (norm_weight(sd, n_embd, norm_type), norm_type)
            else:
                t = types[name]
                qt = t[L % 2] if isinstance(t, tuple) else t
                W[key] = (matrix(sd, qt, *shapes[name]), qt)
    if output_norm:
        W["output_norm.weight"] = (norm_weight(s + 2, n_embd, norm_type), norm_type)
    if not tied:
        W["output.weight"] = (matrix(s + 3, out_type, n_vocab, n_embd), out_type)
    return hp, W


def to_device(W, device="cuda:0"):
    import torch

    return {k: (torch.from_numpy(np.ascontiguousarray(a)).to(device), qt)
            for k, (a, qt) in W.items()}


def q4_0_to_ggml_order(blocks):
    """Q4_0 blocks in jinf's element order (elements 2i, 2i+1 in the low and
    high nibble of qs[i]) -> upstream ggml's (element j low nibble of qs[j],
    element j + 16 its high nibble)."""
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 18).copy()
    qs = b[:, 2:]
    e = np.empty((b.shape[0], 32), np.uint8)
    e[:, 0::2] = qs & 15
    e[:, 1::2] = qs >> 4
    b[:, 2:] = e[:, :16] | (e[:, 16:] << 4)
    return b.reshape(np.shape(blocks))


def write_gguf(path, hp, W, q4_0_ggml_order=False, alignment=32):
    """A GGUF v3 file of the model (llama.* keys, GGUF shapes [cols, rows])."""
    kvs = [("general.architecture", gw.STR, "llama"),
           ("llama.block_count", gw.U32, hp["n_layers"]),
           ("llama.embedding_length", gw.U32, hp["n_embd"]),
           ("llama.attention.head_count", gw.U32, hp["n_heads"]),
           ("llama.attention.head_count_kv", gw.U32, hp["n_heads_kv"]),
           ("llama.feed_forward_length", gw.U32, hp["n_ff"]),
           ("llama.vocab_size", gw.U32, hp["n_vocab"]),
           ("llama.rope.freq_base", gw.F32, hp["rope_freq_base"]),
           ("llama.attention.layer_norm_rms_epsilon", gw.F32, hp["rms_norm_eps"])]
    tensors = []
    for name, (a, qt) in W.items():
        if name.endswith("norm.weight"):
            shape = [a.shape[0]]
        else:
            rows = a.shape[0]
            cols = hp["n_ff"] if name.endswith("ffn_down.weight") else hp["n_embd"]
            shape = [cols, rows]
        data = q4_0_to_ggml_order(a) if (qt == Q4_0 and q4_0_ggml_order) else a
        tensors.append((name, shape, qt, np.ascontiguousarray(data).tobytes()))
    return gw.write(path, kvs, tensors, alignment=alignment)


def gguf_shape(hp, name, a):
    """GGUF dimensions (ne0 = cols first) of a weight of the tiny model."""
    if name.endswith("norm.weight"):
        return [a.shape[0]]
    cols = hp["n_ff"] if name.endswith("ffn_down.weight") else hp["n_embd"]
    return [cols, a.shape[0]]


def _layer_of(name):
    return int(name.split(".")[1]) if name.startswith("blk.") else -1


def write_nvmw(path, hp, W, cold_layers=(), bundled=False, primary_type=None, order=None):
    """A .nvmw file of the model as prepare_model lays it out: the tensors of
    layers in cold_layers in their layer's cold region, everything else hot.
    bundled: also the version-2 neuron bundles (gate row, up row, and the
    down column as fp32, padded to 4 KiB; tools/prepare_model.cpp:296-490).
    order: tensor names in file order (default: W's order)."""
    import nvmw_writer as nw

    names = list(W) if order is None else list(order)
    tensors = []
    for name in names:
        a, qt = W[name]
        L = _layer_of(name)
        tensors.append((name, qt, gguf_shape(hp, name, a), np.ascontiguousarray(a).tobytes(), L,
                        L not in cold_layers))
    if primary_type is None:
        primary_type = W["blk.0.ffn_gate.weight"][1]
    bundles = None
    if bundled:
        n_embd, n_ff = hp["n_embd"], hp["n_ff"]
        bs, bb = oracle.qtype_geometry(primary_type)
        row = (n_embd + bs - 1) // bs * bb
        size = nw.align4k(2 * row + 4 * n_embd)
        per_layer = []
        for L in range(hp["n_layers"]):
            g, gq = W[f"blk.{L}.ffn_gate.weight"]
            u, uq = W[f"blk.{L}.ffn_up.weight"]
            dn, dq = W[f"blk.{L}.ffn_down.weight"]
            gb = np.ascontiguousarray(g).view(np.uint8).reshape(n_ff, -1)
            ub = np.ascontiguousarray(u).view(np.uint8).reshape(n_ff, -1)
            dense = dq in (F32, F16)
            dcol = (dn.astype(np.float32) if dense else oracle.dequant(dq, dn)).reshape(n_embd, n_ff)
            per_layer.append([(gb[j].tobytes() + ub[j].tobytes() +
                               np.ascontiguousarray(dcol[:, j]).tobytes()).ljust(size, b"\0")
                              for j in range(n_ff)])
        bundles = (size, n_ff, per_layer)
    return nw.write(path, hp, tensors, primary_type=primary_type, bundles=bundles)


def pass_through_model(n_vocab=64, n_embd=256):
    """Every layer matrix zero (the residual stream keeps the embedding), an
    output norm keeping only element 0, and an output matrix whose row 2 reads
    element 0: token 2 (end of sequence) wins for every input."""
    hp = dict(n_layers=2, n_embd=n_embd, n_heads=4, n_heads_kv=2, n_ff=256, n_vocab=n_vocab,
              rope_freq_base=10000.0, rms_norm_eps=1e-5)
    kvd = 2 * (n_embd // 4)
    zeros = lambda r, c: (np.zeros((r, c // 32 * 18), np.uint8), Q4_0)  # noqa: E731
    W = {"token_embd.weight": (np.abs(np.random.default_rng(1).normal(size=(n_vocab, n_embd)))
                               .astype(np.float32) + 0.1, F32)}
    shapes = {"attn_q": (n_embd, n_embd), "attn_k": (kvd, n_embd), "attn_v": (kvd, n_embd),
              "attn_output": (n_embd, n_embd), "ffn_gate": (256, n_embd),
              "ffn_up": (256, n_embd), "ffn_down": (n_embd, 256)}
    for L in range(2):
        for n in LAYER_TENSORS:
            W[f"blk.{L}.{n}.weight"] = ((np.ones(n_embd, np.float32), F32) if n.endswith("norm")
                                        else zeros(*shapes[n]))
    g = np.zeros(n_embd, np.float32)
    g[0] = 1.0
    W["output_norm.weight"] = (g, F32)
    out = np.zeros((n_vocab, n_embd // 32, 34), np.uint8)
    out[2, 0, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    out[2, 0, 2] = 1
    W["output.weight"] = (out.reshape(n_vocab, -1), Q8_0)
    return hp, W
