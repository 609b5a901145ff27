"""GPU parity: the decode engine (include/jinf/engine_hip.h) against the
oracle's decode loop (oracle/engine.py, pinned against a float64 textbook
decoder in test_oracle_engine.py) on tiny random models with every weight
format, GQA grouping and KV-cache type.

Bar: after every token, |logits - logits_oracle| <= TOL * max |logits_oracle|
with TOL 1e-4 for an fp32 KV cache.  Each stage of the engine agrees with the
oracle's to within a few fp32 ulps of its operands' scale (the kernels' own
parity tests); the bar leaves room for those differences to pass through two
layers and the attention history (measured: up to 1.4e-5).  With an fp16
cache both sides round K and V to fp16, but a K or V value that differs in
its last fp32 bits can round to the neighbouring fp16 value, a 2^-11
relative step that reaches the logits directly: TOL is 4e-4 there (measured:
up to 4.1e-5).
A wrong position, cache slot, weight row or residual moves the logits by O(1).
The captured graph and the kernel-by-kernel path give identical bits, and
greedy generation reproduces a host-side argmax loop exactly.
"""
import numpy as np
import pytest

import jinf_amd
import model_util as mu
from gpu_util import say
from jinf_amd.engine import Engine, EngineError
from oracle import engine as oeng

pytestmark = pytest.mark.gpu

TOL = 1e-4
TOL_F16_KV = 4e-4

MODELS = {
    # head_dim 64, 4 query heads on 2 kv heads, every block type
    "mixed": dict(),
    # F16 norms, Q4_0 embedding, output tied to the embedding
    "q4_0-f16norm-tied": dict(types={k: mu.Q4_0 for k in mu.MIXED}, norm_type=mu.F16,
                              embd_type=mu.Q4_0, tied=True),
    # head_dim 128, 4 query heads on 1 kv head, F16 embedding table
    "hd128-gqa4": dict(n_embd=512, n_heads=4, n_heads_kv=1, n_ff=512, embd_type=mu.F16),
    # head_dim 96 (generic attention kernel), no output norm, F32 embedding
    "hd96": dict(n_embd=384, n_heads=4, n_heads_kv=2, n_ff=768,
                 types={k: (mu.Q4_0, mu.Q8_0) for k in mu.MIXED}, embd_type=mu.F32,
                 out_type=mu.Q8_0, output_norm=False),
    # q and k of one format, v of another (the Q4_K_M pattern): one Q/K/V
    # launch per format, the second writing only the V rows
    "qk-v-two-formats": dict(types=dict(mu.MIXED, attn_q=(mu.Q4_0, mu.Q4_K),
                                        attn_k=(mu.Q4_0, mu.Q4_K), attn_v=(mu.Q8_0, mu.Q6_K))),
}
TOKENS = [5, 17, 999, 0, 42, 17, 3, 500]


def make_engine(hp, W, max_ctx, kv_type, graph=True):
    e = Engine(hp, mu.to_device(W), max_ctx, kv_type)
    e.use_graph(graph)
    return e


def compare(got, ref, what, tol=TOL):
    scale = float(np.max(np.abs(ref)))
    err = float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64))))
    say(f"{what}: max error / max |logit| = {err / scale:.2e}")
    assert np.all(np.isfinite(got)), what
    assert err <= tol * scale, what


@pytest.mark.parametrize("kv_type", [mu.F32, mu.F16], ids=["kv-f32", "kv-f16"])
@pytest.mark.parametrize("name", list(MODELS))
def test_decode_matches_oracle(dev, name, kv_type):
    say(f"engine decode {name} kv={'f16' if kv_type else 'f32'}")
    hp, W = mu.tiny_model(seed=11, **MODELS[name])
    ref = oeng.Decoder(hp, W, max_context=16, kv_type=kv_type)
    with make_engine(hp, W, 16, kv_type) as e:
        for t, tok in enumerate(TOKENS):
            e.forward([tok])
            assert e.n_past == t + 1
            compare(e.logits(), ref.step(tok), f"{name} token {t}",
                    TOL_F16_KV if kv_type == mu.F16 else TOL)


def test_graph_eager_and_batched_calls_identical(dev):
    say("graph replay vs kernel-by-kernel vs one multi-token call")
    hp, W = mu.tiny_model(seed=12)
    with make_engine(hp, W, 16, mu.F16, graph=True) as g, \
            make_engine(hp, W, 16, mu.F16, graph=False) as k:
        for tok in TOKENS:
            g.forward([tok])
            k.forward([tok])
            assert np.array_equal(g.logits().view(np.uint32), k.logits().view(np.uint32))
        last = g.logits()
        g.reset()
        assert g.n_past == 0
        g.forward(TOKENS)
        assert g.n_past == len(TOKENS)
        assert np.array_equal(g.logits().view(np.uint32), last.view(np.uint32))


def test_long_context_split_attention(dev):
    """fp16 cache over 600 positions: the attention splits the context over
    several workgroups per head; logits checked around the split boundaries."""
    say("engine decode 600 tokens, head_dim 128, fp16 cache")
    hp, W = mu.tiny_model(seed=13, n_embd=512, n_heads=4, n_heads_kv=2, n_ff=512, n_layers=1,
                          n_vocab=512)
    toks = [int(t) for t in np.random.default_rng(13).integers(0, 512, size=600)]
    ref = oeng.Decoder(hp, W, max_context=640, kv_type=mu.F16)
    refs = [ref.step(t) for t in toks]
    with make_engine(hp, W, 640, mu.F16) as e:
        done = 0
        for t in (0, 255, 256, 257, 511, 512, 599):
            e.forward(toks[done:t + 1])
            done = t + 1
            compare(e.logits(), refs[t], f"position {t}", TOL_F16_KV)


def test_generate_matches_host_greedy_loop(dev):
    say("greedy generation vs forward + host argmax")
    hp, W = mu.tiny_model(seed=14, n_vocab=300)
    prompt = [7, 8, 9]
    with make_engine(hp, W, 32, mu.F32) as a, make_engine(hp, W, 32, mu.F32) as b:
        out = a.generate(prompt, 12)
        b.forward(prompt)
        want = []
        for _ in range(12):
            best = oeng.first_argmax(b.logits())
            want.append(best)
            if best == oeng.EOS:
                break
            b.forward([best])
        assert out == want
        assert a.n_past == b.n_past == len(prompt) + len(out) - (out[-1] == oeng.EOS)
        # continuing without a prompt picks up the last step's argmax
        more = a.generate([], 3)
        nxt = oeng.first_argmax(b.logits())
        assert more[0] == nxt
        # the oracle agrees wherever its top-2 gap exceeds the parity bar
        ref = oeng.Decoder(hp, W, max_context=32)
        lg = ref.forward(prompt)
        for tok in out:
            srt = np.sort(lg)[::-1]
            if srt[0] - srt[1] > 2 * TOL * np.max(np.abs(lg)):
                assert tok == oeng.first_argmax(lg)
            lg = ref.step(tok)


@pytest.mark.parametrize("kv_type", [mu.F32, mu.F16], ids=["kv-f32", "kv-f16"])
@pytest.mark.parametrize("name", ["mixed", "q4_0-f16norm-tied", "hd128-gqa4", "hd96"])
def test_prefill_matches_oracle_and_continues(dev, name, kv_type):
    """A prompt through prefill (steps of 64 and 6 tokens on the batched GEMVs
    over the engine's own cache; hd96's n_embd of 384 takes the token-by-token
    path instead) equals the oracle's loop and leaves the engine where
    forward would: later forward steps and greedy generation continue it."""
    max_ctx = 96
    say(f"engine prefill {name} kv={'f16' if kv_type else 'f32'}")
    hp, W = mu.tiny_model(seed=18, **MODELS[name])
    tol = TOL_F16_KV if kv_type == mu.F16 else TOL
    prompt = np.random.default_rng(19).integers(0, hp["n_vocab"], size=70).astype(np.int32)
    ref = oeng.Decoder(hp, W, max_context=max_ctx, kv_type=kv_type)
    with make_engine(hp, W, max_ctx, kv_type) as e:
        e.forward([5])  # the prompt starts at position 1
        ref.step(5)
        e.prefill(prompt)
        for t in prompt:
            want = ref.step(int(t))
        assert e.n_past == 1 + len(prompt)
        compare(e.logits(), want, f"{name} prefill last token", tol)
        for t in (7, 11):
            e.forward([t])
            compare(e.logits(), ref.step(t), f"{name} step after prefill", tol)
        first = oeng.first_argmax(e.logits())
        assert e.generate([], 1) == [first]
        # generation right after a prefill starts from the prompt's argmax
        e.reset()
        e.prefill(prompt[:9])
        nxt = oeng.first_argmax(e.logits())
        assert e.generate([], 1) == [nxt]
        assert e.n_past == 9 + (nxt != oeng.EOS)  # the emitted token was decoded


def test_prefill_errors_and_context_end(dev):
    hp, W = mu.tiny_model(seed=20, n_vocab=64, n_layers=1)
    with make_engine(hp, W, 8, mu.F32) as e:
        for bad in ([64, 1], [1, -1], list(range(9))):
            with pytest.raises(EngineError) as ex:
                e.prefill(bad)
            assert ex.value.status == 5
            assert e.n_past == 0
        e.prefill([3])             # one token: the forward path
        e.prefill(list(range(7)))  # fills the context
        assert e.n_past == 8
        with pytest.raises(EngineError):
            e.prefill([1, 2])
        with pytest.raises(EngineError):
            e.forward([1])
        assert e.generate([], 3) == [oeng.first_argmax(e.logits())]


def test_generate_stops_at_eos(dev):
    say("generation stops after emitting token 2")
    hp, W = mu.pass_through_model()
    with make_engine(hp, W, 16, mu.F32) as e:
        assert e.generate([5, 6], 10) == [oeng.EOS]
        assert e.n_past == 2
        lg = e.logits()
        assert lg[2] > 0 and np.all(np.delete(lg, 2) == 0)


def test_generate_stops_at_context_end(dev):
    say("generation stops when the cache is full")
    hp, W = mu.tiny_model(seed=15, n_vocab=64, n_layers=1)
    ref = oeng.Decoder(hp, W, max_context=6)
    want = ref.generate([1, 2, 3, 4], 10)
    with make_engine(hp, W, 6, mu.F32) as e:
        out = e.generate([1, 2, 3, 4], 10)
        assert len(out) == len(want) and e.n_past == ref.n_past == 6
        with pytest.raises(EngineError) as ex:
            e.forward([1])
        assert ex.value.status == 5


def test_forward_rejects_bad_tokens_and_overflow(dev):
    hp, W = mu.tiny_model(seed=16, n_vocab=64, n_layers=1)
    with make_engine(hp, W, 4, mu.F32) as e:
        for bad in ([64], [-1], [1, 2, 3, 4, 5]):
            with pytest.raises(EngineError) as ex:
                e.forward(bad)
            assert ex.value.status == 5
            assert e.n_past == 0
        with pytest.raises(EngineError):
            e.generate([], 3)        # nothing decoded yet
        e.forward([1, 2, 3, 4])
        assert e.n_past == 4


def test_step_weight_bytes(dev):
    hp, W = mu.tiny_model(seed=17)
    want = sum(a.nbytes for k, (a, _) in W.items() if k != "token_embd.weight")
    emb = W["token_embd.weight"][0]
    want += emb.nbytes // emb.shape[0]
    with make_engine(hp, W, 8, mu.F32) as e:
        assert e.step_weight_bytes == want


def test_engine_stats(dev):
    """jinf_hip_engine_get_stats: the reference's jinf_perf_stats
    (include/jinf/engine.h:14-22) as its forward keeps them (src/engine.cpp:
    756-757): wall time and tokens run through the model, summed over forward,
    prefill and generate calls; the streaming fields stay zero; reset clears."""
    say("engine stats: tokens and wall time per call, cleared by reset")
    hp, W = mu.tiny_model(seed=18, n_vocab=64, n_layers=1)
    with make_engine(hp, W, 32, mu.F32) as e:
        st = e.stats()
        assert st["tokens_generated"] == 0 and st["total_ms"] == 0.0
        e.forward([1, 2, 3])
        st = e.stats()
        assert st["tokens_generated"] == 3 and st["total_ms"] > 0.0
        t0, n0 = st["total_ms"], e.n_past
        e.generate([], 5)                      # every fed-back token counts
        st = e.stats()
        assert st["tokens_generated"] == 3 + (e.n_past - n0) and st["total_ms"] > t0
        n1 = e.n_past
        e.prefill([4, 5, 6, 7])
        st = e.stats()
        assert st["tokens_generated"] == 3 + (n1 - n0) + 4
        for k in ("nvme_read_ms", "gpu_compute_ms", "attention_ms", "ffn_ms", "nvme_bytes_read"):
            assert st[k] == 0.0
        e.reset()
        st = e.stats()
        assert st["tokens_generated"] == 0 and st["total_ms"] == 0.0


@pytest.mark.parametrize("ggml_order", [False, True], ids=["jinf-order", "ggml-order"])
def test_gguf_engine_matches_resident_weights(dev, tmp_path, ggml_order):
    say(f"engine from a GGUF file, Q4_0 in {'ggml' if ggml_order else 'jinf'} order")
    hp, W = mu.tiny_model(seed=18, embd_type=mu.Q4_0)
    path = tmp_path / "tiny.gguf"
    mu.write_gguf(str(path), hp, W, q4_0_ggml_order=ggml_order)
    with make_engine(hp, W, 16, mu.F16) as a, \
            Engine.from_gguf(str(path), 16, mu.F16, q4_0_ggml_order=ggml_order) as b:
        assert b.step_weight_bytes == a.step_weight_bytes
        for tok in TOKENS:
            a.forward([tok])
            b.forward([tok])
            assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))


def test_gguf_missing_tensor(dev, tmp_path):
    hp, W = mu.tiny_model(seed=19, n_layers=1)
    del W["blk.0.ffn_up.weight"]
    path = tmp_path / "broken.gguf"
    mu.write_gguf(str(path), hp, W)
    with pytest.raises(EngineError) as ex:
        Engine.from_gguf(str(path), 16)
    assert ex.value.status == 2


@pytest.mark.parametrize("name", ["mixed", "hd128-gqa4"])
def test_long_prefill_splits_attention_contexts(dev, name):
    """A 330-token prompt through prefill at max_context 512 with an fp16 KV
    cache: the attention of every 64-token step runs over contexts past one
    256-position chunk, so its split contexts are merged -- by the separate
    merge launch when the step has 128 or more (row, head group) pairs
    ("mixed": 64 rows x 2 groups), inside the attention launch otherwise
    (the 10-token last step; "hd128-gqa4": 64 rows x 1 group).  The last
    token's logits and the next decode step equal the oracle's loop."""
    max_ctx = 512
    say(f"engine prefill of 330 tokens, {name}, max_context {max_ctx}, kv f16")
    hp, W = mu.tiny_model(seed=24, **MODELS[name])
    prompt = np.random.default_rng(25).integers(0, hp["n_vocab"], size=330).astype(np.int32)
    ref = oeng.Decoder(hp, W, max_context=max_ctx, kv_type=mu.F16)
    with make_engine(hp, W, max_ctx, mu.F16) as e:
        e.prefill(prompt)
        for t in prompt:
            want = ref.step(int(t))
        assert e.n_past == len(prompt)
        compare(e.logits(), want, f"{name} long prefill last token", TOL_F16_KV)
        e.forward([7])
        compare(e.logits(), ref.step(7), f"{name} step after long prefill", TOL_F16_KV)
