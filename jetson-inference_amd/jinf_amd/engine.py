"""The decode engine of libjinf_hip.so (include/jinf/engine_hip.h): per-token
forward and greedy generation of a Llama-style model whose weights are
resident in device memory (reference src/engine.cpp:684-805).

Weights are named as in GGUF files (``token_embd.weight``,
``blk.N.attn_q.weight``, ..., ``output_norm.weight``, ``output.weight``) and
given as (device tensor, jinf_qtype code) pairs; the tensor holds the raw
blocks (uint8) or F32 / F16 values.
"""
import ctypes

import numpy as np

from ._lib import F16, F32, JINF_HIP_OK, lib

LAYER_TENSORS = ("attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                 "ffn_gate", "ffn_up", "ffn_down")
HPARAMS = ("n_layers", "n_embd", "n_heads", "n_heads_kv", "n_ff", "n_vocab")
EOS = 2


class LayerWeights(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_void_p) for n in LAYER_TENSORS] +
                [(n + "_type", ctypes.c_int32) for n in LAYER_TENSORS])


class EngineDesc(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_heads", ctypes.c_int),
                ("n_heads_kv", ctypes.c_int), ("n_ff", ctypes.c_int), ("n_vocab", ctypes.c_int),
                ("max_context", ctypes.c_int), ("rms_norm_eps", ctypes.c_float),
                ("rope_freq_base", ctypes.c_float), ("kv_type", ctypes.c_int),
                ("token_embd", ctypes.c_void_p), ("token_embd_type", ctypes.c_int32),
                ("output_norm", ctypes.c_void_p), ("output_norm_type", ctypes.c_int32),
                ("output", ctypes.c_void_p), ("output_type", ctypes.c_int32),
                ("layers", ctypes.POINTER(LayerWeights))]


class PerfStats(ctypes.Structure):
    """jinf_hip_perf_stats (include/jinf/engine_hip.h), the reference's
    jinf_perf_stats field for field (include/jinf/engine.h:14-22)."""
    _fields_ = [("total_ms", ctypes.c_double), ("nvme_read_ms", ctypes.c_double),
                ("gpu_compute_ms", ctypes.c_double), ("attention_ms", ctypes.c_double),
                ("ffn_ms", ctypes.c_double), ("tokens_generated", ctypes.c_int),
                ("nvme_bytes_read", ctypes.c_double)]


class EngineError(RuntimeError):
    def __init__(self, what, status):
        super().__init__(f"{what} returned status {status}")
        self.status = status


def _check(what, rc):
    if rc != JINF_HIP_OK:
        raise EngineError(what, rc)


class Engine:
    """A jinf_hip_engine.  Build it from device weights (``Engine(...)``) or
    from a GGUF or .nvmw file (``Engine.from_gguf``, ``Engine.from_nvmw``);
    ``close()`` frees it."""

    def __init__(self, hparams, weights, max_context, kv_type=F32, _handle=None):
        self._keep = []
        if _handle is not None:
            self._h = _handle
            self.n_vocab = hparams["n_vocab"]
            self.max_context = max_context
            return
        d = EngineDesc()
        for k in HPARAMS:
            setattr(d, k, int(hparams[k]))
        d.max_context = int(max_context)
        d.rms_norm_eps = float(hparams.get("rms_norm_eps", 1e-5))
        d.rope_freq_base = float(hparams.get("rope_freq_base", 10000.0))
        d.kv_type = int(kv_type)

        def ptr(name, required=True):
            if name not in weights:
                if required:
                    raise KeyError(name)
                return None, 0
            t, qt = weights[name]
            assert t.is_cuda and t.is_contiguous(), name
            self._keep.append(t)
            return t.data_ptr(), int(qt)

        d.token_embd, d.token_embd_type = ptr("token_embd.weight")
        d.output_norm, d.output_norm_type = ptr("output_norm.weight", False)
        d.output, d.output_type = ptr("output.weight", False)
        layers = (LayerWeights * max(1, d.n_layers))()
        for L in range(d.n_layers):
            for n in LAYER_TENSORS:
                p, qt = ptr(f"blk.{L}.{n}.weight")
                setattr(layers[L], n, p)
                setattr(layers[L], n + "_type", qt)
        d.layers = layers
        h = ctypes.c_void_p()
        _check("jinf_hip_engine_create", lib().jinf_hip_engine_create(ctypes.byref(h),
                                                                      ctypes.byref(d)))
        self._h = h
        self.n_vocab = d.n_vocab
        self.max_context = d.max_context

    @classmethod
    def from_gguf(cls, gguf_file, max_context, kv_type=F16, q4_0_ggml_order=False):
        """gguf_file: a jinf_amd.gguf.GGUFFile (or a path)."""
        from .gguf import GGUFFile

        f = gguf_file if isinstance(gguf_file, GGUFFile) else GGUFFile(gguf_file)
        h = ctypes.c_void_p()
        _check("jinf_hip_engine_create_gguf",
               lib().jinf_hip_engine_create_gguf(ctypes.byref(h), f._h, int(max_context),
                                                 int(kv_type), int(bool(q4_0_ggml_order))))
        return cls(f.hparams, None, max_context, kv_type, _handle=h)

    @classmethod
    def from_nvmw(cls, nvmw_file, max_context, kv_type=F16):
        """nvmw_file: a jinf_amd.nvmw.NVMWFile (or a path)."""
        from .nvmw import NVMWFile

        f = nvmw_file if isinstance(nvmw_file, NVMWFile) else NVMWFile(nvmw_file)
        h = ctypes.c_void_p()
        _check("jinf_hip_engine_create_nvmw",
               lib().jinf_hip_engine_create_nvmw(ctypes.byref(h), f._h, int(max_context),
                                                 int(kv_type)))
        return cls(f.header, None, max_context, kv_type, _handle=h)

    def close(self):
        if getattr(self, "_h", None):
            lib().jinf_hip_engine_destroy(self._h)
            self._h = None
        self._keep = []

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
    def n_past(self):
        return lib().jinf_hip_engine_n_past(self._h)

    def reset(self):
        _check("jinf_hip_engine_reset", lib().jinf_hip_engine_reset(self._h))

    def use_graph(self, on):
        _check("jinf_hip_engine_use_graph", lib().jinf_hip_engine_use_graph(self._h, int(on)))

    @property
    def step_weight_bytes(self):
        return lib().jinf_hip_engine_step_weight_bytes(self._h)

    def stats(self):
        """The engine's counters (jinf_hip_engine_get_stats) as a dict."""
        p = lib().jinf_hip_engine_get_stats(self._h)
        st = PerfStats.from_address(p)
        return {name: getattr(st, name) for name, _ in PerfStats._fields_}

    def forward(self, tokens):
        """Decode `tokens` (ints) one at a time; returns the device address of
        the last token's fp32 logits."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        p = ctypes.c_void_p()
        _check("jinf_hip_engine_forward",
               lib().jinf_hip_engine_forward(self._h, t.ctypes.data, t.size, ctypes.byref(p)))
        return p.value

    def prefill(self, tokens):
        """Decode a prompt in batched steps (jinf_hip_engine_prefill); returns
        the device address of the last token's fp32 logits."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        p = ctypes.c_void_p()
        _check("jinf_hip_engine_prefill",
               lib().jinf_hip_engine_prefill(self._h, t.ctypes.data, t.size, ctypes.byref(p)))
        return p.value

    def logits(self):
        """Host copy (fp32 numpy) of the last token's logits."""
        out = np.empty(self.n_vocab, np.float32)
        _check("jinf_hip_engine_copy_logits",
               lib().jinf_hip_engine_copy_logits(self._h, out.ctypes.data, out.size))
        return out

    def generate(self, prompt, max_tokens):
        """Greedy generation (jinf_hip_engine_generate): the emitted token ids."""
        pr = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32).reshape(-1))
        out = np.zeros(max(1, int(max_tokens)), np.int32)
        n = ctypes.c_int(0)
        _check("jinf_hip_engine_generate",
               lib().jinf_hip_engine_generate(self._h, pr.ctypes.data if pr.size else None,
                                              pr.size, out.ctypes.data, int(max_tokens),
                                              ctypes.byref(n)))
        return [int(x) for x in out[:n.value]]


class Batch:
    """A jinf_hip_batch: n_seq sequences decoded together on an Engine's
    weights (keep the Engine alive while the batch exists)."""

    def __init__(self, engine, n_seq, max_context, kv_type=F16):
        h = ctypes.c_void_p()
        _check("jinf_hip_batch_create",
               lib().jinf_hip_batch_create(ctypes.byref(h), engine._h, int(n_seq),
                                           int(max_context), int(kv_type)))
        self._h = h
        self._engine = engine
        self.n_seq = int(n_seq)
        self.n_vocab = engine.n_vocab
        self.max_context = int(max_context)

    def close(self):
        if getattr(self, "_h", None):
            lib().jinf_hip_batch_destroy(self._h)
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

    def reset(self, seq=-1):
        _check("jinf_hip_batch_reset", lib().jinf_hip_batch_reset(self._h, int(seq)))

    def n_past(self, seq):
        return lib().jinf_hip_batch_n_past(self._h, int(seq))

    def use_graph(self, on=True):
        _check("jinf_hip_batch_use_graph", lib().jinf_hip_batch_use_graph(self._h, int(bool(on))))

    def forward(self, tokens):
        """One step: tokens[s] (-1 = idle) for every sequence."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        if t.size != self.n_seq:
            raise ValueError("one token per sequence")
        p = ctypes.c_void_p()
        _check("jinf_hip_batch_forward",
               lib().jinf_hip_batch_forward(self._h, t.ctypes.data, ctypes.byref(p)))
        return p.value

    def prefill(self, seq, tokens):
        """Sequence seq's prompt in chunks of up to n_seq tokens per step;
        returns the last token's logits, fp32 [n_vocab] (host copy)."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        p = ctypes.c_void_p()
        _check("jinf_hip_batch_prefill",
               lib().jinf_hip_batch_prefill(self._h, int(seq), t.ctypes.data, int(t.size),
                                            ctypes.byref(p)))
        if t.size == 0:
            return None
        return self.logits()[(t.size - 1) % self.n_seq].copy()

    def logits(self):
        """The last step's logits, fp32 [n_seq, n_vocab] (host copy)."""
        out = np.empty((self.n_seq, self.n_vocab), np.float32)
        _check("jinf_hip_batch_copy_logits",
               lib().jinf_hip_batch_copy_logits(self._h, out.ctypes.data))
        return out

    def generate(self, steps):
        """Greedy steps: int32 [steps, n_seq] emitted tokens (-1 after a stop)."""
        out = np.zeros((max(1, int(steps)), self.n_seq), np.int32)
        _check("jinf_hip_batch_generate",
               lib().jinf_hip_batch_generate(self._h, out.ctypes.data, int(steps)))
        return out[:int(steps)]


__all__ = ["Engine", "EngineError", "Batch", "EngineDesc", "LayerWeights", "LAYER_TENSORS", "EOS", "F16",
           "F32"]
