"""GPU parity of the decode engine at Llama-3-8B widths: two layers with
hidden 4096, 32 query / 8 KV heads of 128, FFN 14336 and a 128256-token
vocabulary, in the two weight layouts bench.py times (Q4_0 with a Q6_K output
head, and Q4_K_M: Q4_K with Q6_K for attn_v, ffn_down and the output), fp16
KV cache, checked after each of 4 tokens against the oracle's decode loop
(oracle/engine.py).  The batch decoder at the same widths, in both layouts: 5
and 40 sequences (one and two 32-sequence tiles of the batched GEMVs, whose column
splits are merged by separate launches and whose residual merges hand 2048-
column slice statistics to the normalising preparation), a prompt through
prefill, then decode steps, each sequence against its own oracle loop.

Bar: |logits - logits_oracle| <= 4e-4 * max |logits_oracle| (the fp16-cache
bar of test_gpu_engine.py).  The kernels at these shapes are checked one at a
time by the GEMV, attention and elementwise suites; this checks their
composition by the engine at the real widths (buffer sizes, strides, row
tiling of the 14336-column down projection and the 128256-row output GEMV).
"""
import numpy as np
import pytest

import model_util as mu
import oracle
import testutil as tu
from gpu_util import say
from jinf_amd.engine import Batch, Engine
from oracle import engine as oeng

pytestmark = pytest.mark.gpu

TOL = 4e-4
H, NH, NKV, FF, V = 4096, 32, 8, 14336, 128256


def wide_matrix(seed, qt, rows, cols, rms=None):
    """Random [rows, cols] weight of type qt with dequantized root-mean-square
    about `rms` (default 1/sqrt(cols)), its scale measured on 64 rows."""
    rms = 1.0 / np.sqrt(cols) if rms is None else rms
    probe = tu.quant_table(tu.rng(seed + 7), qt, 64, cols, 0.01)
    got = float(np.sqrt(np.mean(oracle.dequant(qt, probe).astype(np.float64) ** 2)))
    return tu.quant_table(tu.rng(seed), qt, rows, cols, 0.01 * rms / got)


def wide_model(types, embd_type, out_type, seed):
    hp = dict(n_layers=2, n_embd=H, n_heads=NH, n_heads_kv=NKV, n_ff=FF, n_vocab=V,
              rope_freq_base=500000.0, rms_norm_eps=1e-5)
    kvd = NKV * (H // NH)
    shapes = {"attn_q": (H, H), "attn_k": (kvd, H), "attn_v": (kvd, H), "attn_output": (H, H),
              "ffn_gate": (FF, H), "ffn_up": (FF, H), "ffn_down": (H, FF)}
    W = {"token_embd.weight": (wide_matrix(seed, embd_type, V, H, rms=1.0), embd_type)}
    for L in range(2):
        for i, name in enumerate(mu.LAYER_TENSORS):
            key = f"blk.{L}.{name}.weight"
            sd = seed + 10 + 20 * L + i
            if name.endswith("norm"):
                W[key] = (mu.norm_weight(sd, H, mu.F32), mu.F32)
            else:
                W[key] = (wide_matrix(sd, types[name], *shapes[name]), types[name])
    W["output_norm.weight"] = (mu.norm_weight(seed + 2, H, mu.F32), mu.F32)
    W["output.weight"] = (wide_matrix(seed + 3, out_type, V, H), out_type)
    return hp, W


LAYOUTS = {
    "q4_0": (dict.fromkeys(("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                            "ffn_down"), mu.Q4_0), mu.Q4_0, mu.Q6_K),
    "q4_k_m": (dict(attn_q=mu.Q4_K, attn_k=mu.Q4_K, attn_v=mu.Q6_K, attn_output=mu.Q4_K,
                    ffn_gate=mu.Q4_K, ffn_up=mu.Q4_K, ffn_down=mu.Q6_K), mu.Q4_K, mu.Q6_K),
}


@pytest.mark.parametrize("layout", list(LAYOUTS))
def test_llama3_8b_widths_match_oracle(dev, layout):
    types, embd_type, out_type = LAYOUTS[layout]
    say(f"2-layer Llama-3-8B-wide model, {layout}, fp16 KV cache, 4 tokens")
    hp, W = wide_model(types, embd_type, out_type, seed=4096 + len(layout))
    ref = oeng.Decoder(hp, W, max_context=16, kv_type=mu.F16)
    oracle.set_threads(16)
    try:
        with Engine(hp, mu.to_device(W), 16, mu.F16) as e:
            for i, tok in enumerate((128000, 9906, 1917, 127999)):
                e.forward([tok])
                got, want = e.logits(), ref.step(tok)
                scale = float(np.max(np.abs(want)))
                err = float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64))))
                say(f"{layout} token {i}: max error / max |logit| = {err / scale:.2e}")
                assert np.all(np.isfinite(got))
                assert err <= TOL * scale, f"{layout} token {i}"
    finally:
        oracle.set_threads(1)


STREAMS = [(128000, 9906, 1917), (128000, 40, 3), (5, 6, 7)]


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("n_seq", [5, 40])
def test_llama3_8b_widths_batch_decode(dev, n_seq, layout):
    """Sequence s decodes STREAMS[s % 3] after sequence 0 took a 6-token prompt
    through prefill; sequences of one stream must agree with that stream's
    oracle loop (and so with each other), sequence 0 with its own.  The
    Q4_K_M layout mixes formats within the Q/K/V projections (Q4_K q and k,
    Q6_K v share one x preparation) and puts the 14336-column down projection
    and the 128256-row output head in Q6_K; 40 sequences take the batched
    GEMVs' second 32-sequence tile."""
    types, embd_type, out_type = LAYOUTS[layout]
    say(f"2-layer Llama-3-8B-wide model, {layout}, batch of {n_seq}, fp16 KV cache")
    hp, W = wide_model(types, embd_type, out_type, seed=8192 + n_seq + 97 * len(layout))
    prompt = (128000, 791, 6864, 315, 9822, 374)
    refs = [oeng.Decoder(hp, W, max_context=16, kv_type=mu.F16) for _ in STREAMS]
    ref0 = oeng.Decoder(hp, W, max_context=16, kv_type=mu.F16)
    oracle.set_threads(16)
    try:
        with Engine(hp, mu.to_device(W), 16, mu.F16) as e, Batch(e, n_seq, 16, mu.F16) as b:
            got = b.prefill(0, prompt)
            for tok in prompt:
                want = ref0.step(tok)
            check_logits(got, want, f"batch {n_seq} prefill")
            for k in range(3):
                row = np.array([STREAMS[s % 3][k] for s in range(n_seq)], np.int32)
                b.forward(row)
                lg = b.logits()
                want = [r.step(st[k]) for r, st in zip(refs, STREAMS)]
                want0 = ref0.step(int(row[0]))
                check_logits(lg[0], want0, f"batch {n_seq} step {k} seq 0")
                for s in range(1, n_seq):
                    check_logits(lg[s], want[s % 3], f"batch {n_seq} step {k} seq {s}", quiet=s > 3)
    finally:
        oracle.set_threads(1)


def check_logits(got, want, what, quiet=False):
    scale = float(np.max(np.abs(want)))
    err = float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64))))
    if not quiet:
        say(f"{what}: max error / max |logit| = {err / scale:.2e}")
    assert np.all(np.isfinite(got)), what
    assert err <= TOL * scale, f"{what}: {err / scale:.2e}"
