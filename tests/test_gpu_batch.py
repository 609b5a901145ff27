"""GPU parity: batched decode (include/jinf/engine_hip.h jinf_hip_batch_*) --
several sequences decoded together on one engine's weights, each with its
own position and KV-cache region -- against the oracle's one-sequence decode
loop (oracle/engine.py, pinned in test_oracle_engine.py) run separately for
every sequence on that sequence's own tokens.

Bars as in test_gpu_engine.py: after every step, each decoding sequence's
logits within TOL (fp32 cache) / TOL_F16_KV (fp16 cache) of the logit scale;
the batched GEMVs keep about 22 bits of x (far inside these bars).  Idle
steps (id -1), ragged prompts, resets of one sequence, graph vs eager
replays (bit-exact) and greedy generation (exactly the host argmax loop over
the batch's own logits, with end-of-sequence and full-context stops) are
covered, and batches of 33-64 sequences (two 32-token tiles)."""
import numpy as np
import pytest

import model_util as mu
from gpu_util import say
from jinf_amd.engine import Batch, Engine, EngineError
from oracle import engine as oeng

pytestmark = pytest.mark.gpu

TOL = 1e-4
TOL_F16_KV = 4e-4

MODELS = {
    "mixed": dict(),
    "q4_0-f16norm-tied": dict(types={k: mu.Q4_0 for k in mu.MIXED}, norm_type=mu.F16,
                              embd_type=mu.Q4_0, tied=True),
    "hd128-gqa4-f16embd": dict(n_embd=512, n_heads=4, n_heads_kv=1, n_ff=512, embd_type=mu.F16),
    "k-quants-f32embd": dict(types={k: (mu.Q4_K, mu.Q6_K) for k in mu.MIXED}, embd_type=mu.F32,
                             out_type=mu.Q8_0, output_norm=False),
}


def compare(got, ref, what, tol):
    scale = float(np.max(np.abs(ref)))
    err = float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64))))
    assert np.all(np.isfinite(got)), what
    assert err <= tol * scale, f"{what}: {err / scale:.2e}"
    return err / scale


def streams(seed, n_seq, n_steps, n_vocab, idle=0.25):
    """Per step, one id per sequence (-1 = idle)."""
    r = np.random.default_rng(seed)
    T = r.integers(0, n_vocab, size=(n_steps, n_seq)).astype(np.int32)
    T[r.random(size=T.shape) < idle] = -1
    return T


@pytest.mark.parametrize("kv_type", [mu.F32, mu.F16], ids=["kv-f32", "kv-f16"])
@pytest.mark.parametrize("name", list(MODELS))
def test_batch_matches_oracle_per_sequence(dev, name, kv_type):
    n_seq, n_steps, max_ctx = 5, 9, 16
    say(f"batch decode {name} kv={'f16' if kv_type else 'f32'} n_seq={n_seq}")
    hp, W = mu.tiny_model(seed=51, n_vocab=400, **MODELS[name])
    refs = [oeng.Decoder(hp, W, max_context=max_ctx, kv_type=kv_type) for _ in range(n_seq)]
    T = streams(52, n_seq, n_steps, hp["n_vocab"])
    tol = TOL_F16_KV if kv_type == mu.F16 else TOL
    worst = 0.0
    with Engine(hp, mu.to_device(W), 8, kv_type) as e, Batch(e, n_seq, max_ctx, kv_type) as b:
        for k, row in enumerate(T):
            b.forward(row)
            lg = b.logits()
            for s, tok in enumerate(row):
                if tok < 0:
                    continue
                worst = max(worst, compare(lg[s], refs[s].step(int(tok)), f"step {k} seq {s}", tol))
            for s in range(n_seq):
                assert b.n_past(s) == int(np.sum(T[:k + 1, s] >= 0))
    say(f"worst error / logit scale {worst:.2e}")


@pytest.mark.parametrize("n_seq", [33, 64])
def test_wide_batches(dev, n_seq):
    """More than 32 sequences: the GEMVs' second token tile."""
    say(f"batch decode n_seq={n_seq}")
    hp, W = mu.tiny_model(seed=53, n_vocab=300)
    refs = [oeng.Decoder(hp, W, max_context=8, kv_type=mu.F16) for _ in range(n_seq)]
    T = streams(54, n_seq, 4, hp["n_vocab"], idle=0.1)
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e, Batch(e, n_seq, 8, mu.F16) as b:
        for k, row in enumerate(T):
            b.forward(row)
            lg = b.logits()
            for s, tok in enumerate(row):
                if tok >= 0:
                    compare(lg[s], refs[s].step(int(tok)), f"step {k} seq {s}", TOL_F16_KV)


def test_graph_eager_identical_and_reset_one_sequence(dev):
    hp, W = mu.tiny_model(seed=55, n_vocab=300)
    T = streams(56, 4, 6, hp["n_vocab"], idle=0.0)
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e, Batch(e, 4, 16, mu.F16) as g, \
            Batch(e, 4, 16, mu.F16) as k:
        k.use_graph(False)
        outs = []
        for row in T:
            g.forward(row)
            k.forward(row)
            a, c = g.logits(), k.logits()
            assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
            outs.append(a)
        # sequence 2 starts over: replaying its tokens (others idle) gives the same bits
        g.reset(2)
        assert g.n_past(2) == 0 and g.n_past(1) == len(T)
        for t, row in enumerate(T):
            only = np.full(4, -1, np.int32)
            only[2] = row[2]
            g.forward(only)
            assert np.array_equal(g.logits()[2].view(np.uint32), outs[t][2].view(np.uint32))
        assert g.n_past(2) == len(T) and g.n_past(0) == len(T)


def host_greedy(e, prompts, steps, max_ctx, kv_type):
    """Ragged prompts through forward (shorter ones idle), then the host loop:
    emit each sequence's last argmax, decode it unless it is the end of
    sequence or the context is full."""
    n_seq = len(prompts)
    want = np.full((steps, n_seq), -1, np.int32)
    with Batch(e, n_seq, max_ctx, kv_type) as c:
        cur = [None] * n_seq
        for k in range(max(len(p) for p in prompts)):
            row = [p[k] if k < len(p) else -1 for p in prompts]
            c.forward(row)
            L = c.logits()
            for s, p in enumerate(prompts):
                if k == len(p) - 1:
                    cur[s] = oeng.first_argmax(L[s])
        live = [True] * n_seq
        for t in range(steps):
            row = [-1] * n_seq
            for s in range(n_seq):
                if not live[s]:
                    continue
                want[t, s] = cur[s]
                if cur[s] == oeng.EOS or c.n_past(s) >= max_ctx:
                    live[s] = False
                else:
                    row[s] = cur[s]
            if all(r < 0 for r in row):
                continue
            c.forward(row)
            L = c.logits()
            for s in range(n_seq):
                if row[s] >= 0:
                    cur[s] = oeng.first_argmax(L[s])
    return want


def run_generate(e, prompts, steps, max_ctx, kv_type):
    n_seq = len(prompts)
    with Batch(e, n_seq, max_ctx, kv_type) as a:
        for k in range(max(len(p) for p in prompts)):
            a.forward([p[k] if k < len(p) else -1 for p in prompts])
        out = a.generate(steps)
        return out, [a.n_past(s) for s in range(n_seq)]


def test_generate_matches_host_greedy_loop(dev):
    say("batch greedy generation vs forward + host argmax")
    hp, W = mu.tiny_model(seed=57, n_vocab=300)
    prompts = [[7, 8, 9], [4], [100, 200], [5, 6, 7, 8]]
    with Engine(hp, mu.to_device(W), 8, mu.F32) as e:
        out, _ = run_generate(e, prompts, 10, 32, mu.F32)
        want = host_greedy(e, prompts, 10, 32, mu.F32)
    assert np.array_equal(out, want), (out, want)


def test_generate_stops_at_eos_and_context_end(dev):
    # every argmax is the end-of-sequence id: emitted once, then -1
    hp, W = mu.pass_through_model()
    with Engine(hp, mu.to_device(W), 8, mu.F32) as e:
        out, n_past = run_generate(e, [[5, 6], [7]], 4, 16, mu.F32)
        assert out[:, 0].tolist() == [oeng.EOS, -1, -1, -1] and n_past == [2, 1]
        assert out[:, 1].tolist() == [oeng.EOS, -1, -1, -1]
    # full contexts: sequence 0 (2 of 3 positions used) emits, decodes, emits, stops
    hp, W = mu.tiny_model(seed=58, n_vocab=300)
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e:
        out, n_past = run_generate(e, [[5, 7], [6]], 4, 3, mu.F16)
        want = host_greedy(e, [[5, 7], [6]], 4, 3, mu.F16)
        assert np.array_equal(out, want), (out, want)
        assert out[2, 0] == -1 and n_past == [3, 3]
        with Batch(e, 2, 3, mu.F16) as b:
            b.forward([5, 6])
            b.forward([7, -1])
            b.forward([8, -1])
            with pytest.raises(EngineError) as ex:
                b.forward([1, -1])  # sequence 0's context is full
            assert ex.value.status == 5
            with pytest.raises(EngineError):
                b.forward([300, -1])  # id outside the vocabulary


def test_batch_rejects_shapes(dev):
    hp, W = mu.tiny_model(seed=59, n_embd=384, n_heads=4, n_heads_kv=2, n_ff=768,
                          types={k: (mu.Q4_0, mu.Q8_0) for k in mu.MIXED}, embd_type=mu.Q4_0,
                          out_type=mu.Q8_0)
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e:
        with pytest.raises(EngineError) as ex:
            Batch(e, 2, 8, mu.F16)  # n_embd not a multiple of 256
        assert ex.value.status == 5
        with pytest.raises(EngineError):
            Batch(e, 65, 8, mu.F16)


@pytest.mark.parametrize("kv_type", [mu.F32, mu.F16], ids=["kv-f32", "kv-f16"])
@pytest.mark.parametrize("name", ["mixed", "hd128-gqa4-f16embd"])
def test_prefill_matches_oracle_and_continues(dev, name, kv_type):
    """A prompt through prefill (chunks of n_seq tokens sharing one KV region)
    equals the oracle's token-by-token loop, leaves the sequence where that
    loop would, and does not touch the other sequences."""
    n_seq, max_ctx = 4, 24
    say(f"batch prefill {name} kv={'f16' if kv_type else 'f32'}")
    hp, W = mu.tiny_model(seed=61, n_vocab=350, **MODELS[name])
    tol = TOL_F16_KV if kv_type == mu.F16 else TOL
    r = np.random.default_rng(62)
    prompt = r.integers(0, hp["n_vocab"], size=11).astype(np.int32)  # chunks 4, 4, 3
    ref = oeng.Decoder(hp, W, max_context=max_ctx, kv_type=kv_type)
    for t in prompt:
        want = ref.step(int(t))
    other = oeng.Decoder(hp, W, max_context=max_ctx, kv_type=kv_type)
    with Engine(hp, mu.to_device(W), 8, kv_type) as e, Batch(e, n_seq, max_ctx, kv_type) as b:
        b.forward([5, -1, -1, -1])  # sequence 0 has one token already
        other.step(5)
        got = b.prefill(2, prompt)
        compare(got, want, "prefill last token", tol)
        assert [b.n_past(s) for s in range(n_seq)] == [1, 0, len(prompt), 0]
        # the next steps continue both sequences from where they are
        for k, (t0, t2) in enumerate([(7, 9), (11, 13)]):
            b.forward([t0, -1, t2, -1])
            lg = b.logits()
            compare(lg[0], other.step(t0), f"step {k} seq 0", tol)
            compare(lg[2], ref.step(t2), f"step {k} seq 2", tol)
        # greedy generation starts from the prompt's own argmax
        first = oeng.first_argmax(lg[2])
        out = b.generate(1)
        assert out[0, 2] == first


def test_prefill_argmax_and_errors(dev):
    hp, W = mu.tiny_model(seed=63, n_vocab=300)
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e, Batch(e, 3, 10, mu.F16) as b:
        got = b.prefill(1, [3, 4, 5, 6, 7])
        out = b.generate(1)
        assert out[0, 1] == oeng.first_argmax(got)
        assert out[0, 0] == -1 and out[0, 2] == -1  # no token yet: idle
        with pytest.raises(EngineError) as ex:
            b.prefill(1, [1] * 5)  # 6 of 10 used: 5 more do not fit
        assert ex.value.status == 5
        with pytest.raises(EngineError):
            b.prefill(0, [300])  # id outside the vocabulary
        with pytest.raises(EngineError):
            b.prefill(3, [1])  # no such sequence
        assert b.prefill(0, []) is None and b.n_past(0) == 0


def test_prefill_wide_chunks(dev):
    """Chunks of more than 32 prompt tokens (the GEMVs' second token tile)."""
    n_seq, max_ctx = 40, 64
    hp, W = mu.tiny_model(seed=64, n_vocab=300)
    prompt = np.random.default_rng(65).integers(0, hp["n_vocab"], size=45).astype(np.int32)
    ref = oeng.Decoder(hp, W, max_context=max_ctx, kv_type=mu.F16)
    for t in prompt:
        want = ref.step(int(t))
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e, Batch(e, n_seq, max_ctx, mu.F16) as b:
        got = b.prefill(7, prompt)  # chunks of 40 and 5 tokens
        compare(got, want, "prefill last token", TOL_F16_KV)
        assert b.n_past(7) == 45
        row = np.full(n_seq, -1, np.int32)
        row[7] = 3
        b.forward(row)
        compare(b.logits()[7], ref.step(3), "after prefill", TOL_F16_KV)


@pytest.mark.parametrize("name", ["mixed", "hd128-gqa4-f16embd"])
def test_long_prefill_splits_attention_contexts(dev, name):
    """A 330-token prompt through the batch decoder's prefill (chunks of 64
    tokens, one per sequence slot, sharing one KV region) at max_context 512
    with an fp16 cache: contexts past 256 positions are split and merged by
    the separate merge launch (64 rows x 2 head groups in "mixed") or inside
    the attention launch (the 10-token last chunk; 64 x 1 groups in the
    other model).  The last token's logits and the next step of that
    sequence equal the oracle's loop."""
    n_seq, max_ctx = 64, 512
    say(f"batch prefill of 330 tokens, {name}, max_context {max_ctx}, kv f16")
    hp, W = mu.tiny_model(seed=66, n_vocab=350, **MODELS[name])
    prompt = np.random.default_rng(67).integers(0, hp["n_vocab"], size=330).astype(np.int32)
    ref = oeng.Decoder(hp, W, max_context=max_ctx, kv_type=mu.F16)
    for t in prompt:
        want = ref.step(int(t))
    with Engine(hp, mu.to_device(W), 8, mu.F16) as e, Batch(e, n_seq, max_ctx, mu.F16) as b:
        got = b.prefill(5, prompt)
        compare(got, want, "long prefill last token", TOL_F16_KV)
        assert b.n_past(5) == len(prompt)
        row = np.full(n_seq, -1, np.int32)
        row[5] = 7
        b.forward(row)
        compare(b.logits()[5], ref.step(7), "step after long prefill", TOL_F16_KV)
