// jinf decode engine: the reference's per-token forward loop
// (src/engine.cpp:684-760, per layer :418-511, greedy generation :762-805)
// on this library's kernels, weights resident in device memory.
//
// The position of the token being decoded lives in device memory (`state`),
// together with the attention length, the token id, the last argmax and the
// end of the host-provided tokens.  Every kernel of a step reads the position
// from there, so one captured HIP graph decodes every token: the step's last
// kernel advances the position and stores the argmax as the next token, and
// the host keeps its own count of n_past alongside.
//
// Buffers (fp32 activations, as in the reference's scratch_a / scratch_b /
// hidden_buf / logits_buf, src/engine.cpp:196-208) live in one allocation;
// the K and V caches in another, layer-major [n_layers][max_ctx][kv_dim].

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <functional>
#include <new>
#include <string>
#include <vector>

#include "jinf/engine_api.h"
#include "jinf/engine_hip.h"
#include "jinf_device.h"
#include "jinf_host.h"
#include "quant_device.h"
#include "argmax_device.h"
#include "engine_internal.h"

namespace jinf {
namespace {

// Words of the device state block.
enum { kPos = 0, kLen = 1, kTok = 2, kBest = 3, kFillEnd = 4, kStateWords = 64 };
constexpr int kEos = 2;            // end-of-sequence id (src/engine.cpp:796-797)
constexpr int kArgMaxParts = 256;
constexpr int kPrefillRows = 64;   // prompt tokens per batched prefill step
constexpr size_t kAlign = 256;

// Step prologue: the token at the current position, and the attention length
// n_past + 1 (src/engine.cpp:446-456).
__global__ void eng_begin_kernel(int32_t* __restrict__ st, const int32_t* __restrict__ tokens,
                                 int max_ctx) {
    if (threadIdx.x != 0) return;
    const int pos = st[kPos];
    st[kLen] = pos + 1;
    st[kTok] = (pos >= 0 && pos < max_ctx) ? tokens[pos] : -1;
}

// Embedding row of an F32 table (the reference's device copy,
// src/engine.cpp:327-330) or an F16 table (widened exactly); an id outside
// [0, n_vocab) gives zeros.
template <typename T>
__global__ __launch_bounds__(256) void eng_embed_dense_kernel(float* __restrict__ out,
                                                              const T* __restrict__ table,
                                                              const int32_t* __restrict__ st,
                                                              int n_vocab, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int id = st[kTok];
    float v = 0.0f;
    if (id >= 0 && id < n_vocab) {
        if constexpr (sizeof(T) == 2)
            v = h2f(table[(int64_t)id * n + i]);
        else
            v = table[(int64_t)id * n + i];
    }
    out[i] = v;
}

// Greedy argmax, part 1: each workgroup's best over a strided slice.
__global__ __launch_bounds__(kArgThreads) void eng_argmax_part_kernel(const float* __restrict__ x,
                                                                      int n,
                                                                      float* __restrict__ pv,
                                                                      int* __restrict__ pi) {
    float bv = -INFINITY;
    int bi = n;
    for (int j = blockIdx.x * kArgThreads + threadIdx.x; j < n; j += gridDim.x * kArgThreads)
        take(bv, bi, x[j], j);
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

// Greedy argmax, part 2, and the end of the step.  The reference scans the
// logits from element 0 keeping strict improvements (src/engine.cpp:783-791):
// the result is the first index of the largest value, NaNs after element 0
// are skipped, and a NaN element 0 is never improved on.  The result becomes
// the token at the next position unless the host provided that token, and
// the position advances (n_past++, src/engine.cpp:749).
__global__ __launch_bounds__(kArgThreads) void eng_argmax_end_kernel(
    const float* __restrict__ x, int n, const float* __restrict__ pv, const int* __restrict__ pi,
    int parts, int32_t* __restrict__ st, int32_t* __restrict__ tokens, int max_ctx) {
    float bv = -INFINITY;
    int bi = n;
    for (int k = threadIdx.x; k < parts; k += kArgThreads) take(bv, bi, pv[k], pi[k]);
    block_best(bv, bi);
    if (threadIdx.x != 0) return;
    const int best = (__builtin_isnan(x[0]) || bi >= n) ? 0 : bi;
    const int pos = st[kPos];
    st[kBest] = best;
    if (pos + 1 < max_ctx && pos + 1 >= st[kFillEnd]) tokens[pos + 1] = best;
    st[kPos] = pos + 1;
}

// End of a prefill: the state n_tokens forward steps leave (position
// new_pos, last argmax `best`, which is also the token at new_pos).
__global__ void eng_prefill_end_kernel(int32_t* __restrict__ st, int32_t* __restrict__ tokens,
                                       const int32_t* __restrict__ best, int new_pos,
                                       int max_ctx) {
    if (threadIdx.x != 0) return;
    const int b = *best;
    st[kPos] = new_pos;
    st[kBest] = b;
    st[kFillEnd] = new_pos;
    if (new_pos < max_ctx) tokens[new_pos] = b;
}

bool is_matrix_type(int t) { return t == kQ4_0 || t == kQ8_0 || t == kQ4_K || t == kQ6_K; }
bool is_dense_type(int t) { return t == JINF_HIP_F32 || t == JINF_HIP_F16; }

// Values per block and bytes per block of a weight type (dense: 1 value).
void geometry(int t, int* elems, int* bytes) {
    switch (t) {
        case JINF_HIP_F32: *elems = 1; *bytes = 4; return;
        case JINF_HIP_F16: *elems = 1; *bytes = 2; return;
        case kQ4_0: *elems = 32; *bytes = 18; return;
        case kQ8_0: *elems = 32; *bytes = 34; return;
        case kQ4_K: *elems = 256; *bytes = 144; return;
        case kQ6_K: *elems = 256; *bytes = 210; return;
        default: *elems = 0; *bytes = 0; return;
    }
}

// Bytes of a [rows, cols] weight of type t (0 when cols is not whole blocks).
uint64_t weight_bytes(int t, int64_t rows, int64_t cols) {
    int e, b;
    geometry(t, &e, &b);
    if (e == 0 || cols % e != 0) return 0;
    return (uint64_t)rows * (uint64_t)(cols / e) * (uint64_t)b;
}

size_t up_to(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace
}  // namespace jinf

using namespace jinf;

struct jinf_hip_engine {
    jinf_hip_engine_desc d{};
    std::vector<jinf_hip_layer_weights> layers;
    int head_dim = 0, q_dim = 0, kv_dim = 0, kv_es = 4;
    int n_past = 0;
    int arg_parts = 1;
    void* owned_weights = nullptr;  // the GGUF constructor's upload
    char* act = nullptr;            // activations, argmax partials, tokens, state
    char* kv = nullptr;             // K caches, then V caches
    size_t kv_layer_bytes = 0;
    float *hidden = nullptr, *q = nullptr, *attn = nullptr, *gate = nullptr, *up = nullptr;
    float* logits = nullptr;
    float* part_v = nullptr;
    int32_t *part_i = nullptr, *tokens = nullptr, *state = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    int32_t* h_tokens = nullptr;  // pinned staging: max_ctx token ids, then one word
    hipStream_t stream = nullptr;
    // captured token steps, one per attention bound (a power of two >= 64,
    // at most max_context): the bound sets the attention's launch geometry
    // and must cover every length the step can see
    std::vector<std::pair<int, hipGraphExec_t>> graphs;
    int bound = 0;
    bool use_graph = true;
    // prompt path: a batch over this engine's cache, made on the first
    // prefill call (pre_state 1), or -1 when the model's shape is one the
    // batched GEMVs do not take
    jinf_hip_batch* pre = nullptr;
    int pre_state = 0;
    jinf_hip_perf_stats perf{};  // host wall time and tokens of the calls
};

namespace {

#define ENG_TRY(expr)                         \
    do {                                      \
        const int rc_ = (expr);               \
        if (rc_ != JINF_HIP_OK) return rc_;   \
    } while (0)

int hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return JINF_HIP_OK;
    JINF_LOG("engine: %s failed: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? JINF_HIP_ERR_OOM : JINF_HIP_ERR_DEVICE;
}

// Embedding gather for the token in state[kTok] (src/engine.cpp:311-334).
int enqueue_embed(jinf_hip_engine* e) {
    const jinf_hip_engine_desc& d = e->d;
    if (d.token_embd_type == JINF_HIP_F32)
        return launch(eng_embed_dense_kernel<float>, dim3((d.n_embd + 255) / 256), dim3(256), 0,
                      e->stream, e->hidden, static_cast<const float*>(d.token_embd), e->state,
                      d.n_vocab, d.n_embd);
    if (d.token_embd_type == JINF_HIP_F16)
        return launch(eng_embed_dense_kernel<uint16_t>, dim3((d.n_embd + 255) / 256), dim3(256),
                      0, e->stream, e->hidden, static_cast<const uint16_t*>(d.token_embd),
                      e->state, d.n_vocab, d.n_embd);
    // the block-format gather takes the id array itself: the state's token word
    return jinf_dequant_rows(e->hidden, d.n_embd, d.token_embd, d.token_embd_type, d.n_vocab,
                             d.n_embd, e->state + kTok, 1, JINF_HIP_F32, e->stream);
}

// Q, K and V projections of one layer with their RMSNorm, RoPE and cache
// stores; matrices of one weight format share a launch, and q and k of one
// format with v of another (Q4_K_M) share one as well where the shapes allow.
int enqueue_qkv(jinf_hip_engine* e, const jinf_hip_layer_weights& w, void* kc, void* vc) {
    const jinf_hip_engine_desc& d = e->d;
    const void* W[3] = {w.attn_q, w.attn_k, w.attn_v};
    const int T[3] = {w.attn_q_type, w.attn_k_type, w.attn_v_type};
    if (T[0] == T[1] && T[2] != T[0] && w.attn_norm) {
        bool launched = false;
        ENG_TRY(rmsnorm_qkv_rope_two(W[0], W[1], T[0], W[2], T[2], e->hidden, w.attn_norm,
                                     w.attn_norm_type, d.rms_norm_eps, d.n_embd, e->q, kc, vc,
                                     d.kv_type, e->state + kPos, d.max_context, e->head_dim,
                                     d.n_heads, d.n_heads_kv, d.rope_freq_base, e->stream,
                                     &launched));
        if (launched) return JINF_HIP_OK;
    }
    bool done[3] = {false, false, false};
    for (int i = 0; i < 3; ++i) {
        if (done[i]) continue;
        const void* p[3] = {nullptr, nullptr, nullptr};
        for (int j = i; j < 3; ++j)
            if (!done[j] && T[j] == T[i]) {
                p[j] = W[j];
                done[j] = true;
            }
        ENG_TRY(jinf_rmsnorm_qkv_rope(p[0], p[1], p[2], T[i], e->hidden, w.attn_norm,
                                      w.attn_norm_type, d.rms_norm_eps, d.n_embd, e->q, kc, vc,
                                      d.kv_type, e->state + kPos, d.max_context, e->head_dim,
                                      d.n_heads, d.n_heads_kv, d.rope_freq_base, e->stream));
    }
    return JINF_HIP_OK;
}

// One token step: every launch of src/engine.cpp:692-749 for a model whose
// layers are all resident.  Each RMSNorm runs inside the GEMVs that read its
// output, each residual add inside the GEMV that produces its addend, RoPE
// and the cache stores inside the Q/K/V GEMV, SiLU * up inside the gate/up
// GEMV: per layer one Q/K/V launch (more when the three use different
// formats), attention, and three GEMVs.
int enqueue_step(jinf_hip_engine* e) {
    const jinf_hip_engine_desc& d = e->d;
    hipStream_t s = e->stream;
    const int n = d.n_embd, nff = d.n_ff, hd = e->head_dim, qd = e->q_dim, kvd = e->kv_dim;
    const float eps = d.rms_norm_eps;
    ENG_TRY(launch(eng_begin_kernel, dim3(1), dim3(64), 0, s, e->state, e->tokens,
                   d.max_context));
    ENG_TRY(enqueue_embed(e));
    for (int L = 0; L < d.n_layers; ++L) {
        const jinf_hip_layer_weights& w = e->layers[L];
        char* kc = e->kv + (size_t)L * e->kv_layer_bytes;
        char* vc = e->kv + (size_t)(d.n_layers + L) * e->kv_layer_bytes;
        // attention RMSNorm, Q/K/V projections, RoPE at n_past and the K/V
        // cache rows (:429-453): one launch per distinct weight format
        ENG_TRY(enqueue_qkv(e, w, kc, vc));
        // attention over n_past + 1 positions (:455-459)
        ENG_TRY(jinf_attention_decode(e->attn, qd, e->q, qd, kc, vc, d.kv_type, kvd,
                                      (int64_t)d.max_context * kvd, e->state + kLen, 1,
                                      e->bound, hd, d.n_heads, d.n_heads_kv, 0.0f, e->ws,
                                      e->ws_bytes, s));
        // output projection + residual add (:461-466)
        ENG_TRY(jinf_matvec_add(w.attn_output, w.attn_output_type, e->attn, e->hidden, n, qd, s));
        // FFN RMSNorm, gate and up projections, SiLU * up (:487-502)
        if (w.ffn_gate_type == w.ffn_up_type) {
            ENG_TRY(jinf_rmsnorm_swiglu_matvec(w.ffn_gate, w.ffn_up, w.ffn_gate_type, e->hidden,
                                               w.ffn_norm, w.ffn_norm_type, eps, e->gate, nff, n,
                                               s));
        } else {
            ENG_TRY(jinf_rmsnorm_matvec(w.ffn_gate, w.ffn_gate_type, e->hidden, w.ffn_norm,
                                        w.ffn_norm_type, eps, e->gate, nff, n, s));
            ENG_TRY(jinf_rmsnorm_matvec(w.ffn_up, w.ffn_up_type, e->hidden, w.ffn_norm,
                                        w.ffn_norm_type, eps, e->up, nff, n, s));
            ENG_TRY(jinf_swiglu_rows(e->gate, nff, e->gate, nff, e->up, nff, 1, nff,
                                     JINF_HIP_F32, s));
        }
        // down projection + residual add (:504-508)
        ENG_TRY(jinf_matvec_add(w.ffn_down, w.ffn_down_type, e->gate, e->hidden, n, nff, s));
    }
    // final RMSNorm (:736-741) and output projection (:743-747)
    ENG_TRY(jinf_rmsnorm_matvec(d.output, d.output_type, e->hidden, d.output_norm,
                                d.output_norm_type, eps, e->logits, d.n_vocab, n, s));
    // greedy argmax, next token, position advance (:780-800)
    ENG_TRY(launch(eng_argmax_part_kernel, dim3(e->arg_parts), dim3(kArgThreads), 0, s,
                   e->logits, d.n_vocab, e->part_v, e->part_i));
    return launch(eng_argmax_end_kernel, dim3(1), dim3(kArgThreads), 0, s, e->logits, d.n_vocab,
                  e->part_v, e->part_i, e->arg_parts, e->state, e->tokens, d.max_context);
}

int capture(jinf_hip_engine* e, hipGraphExec_t* out) {
    ENG_TRY(hip_ok(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal),
                   "hipStreamBeginCapture"));
    const int rc = enqueue_step(e);
    hipGraph_t g = nullptr;
    const int ec = hip_ok(hipStreamEndCapture(e->stream, &g), "hipStreamEndCapture");
    if (rc != JINF_HIP_OK || ec != JINF_HIP_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc != JINF_HIP_OK ? rc : ec;
    }
    hipGraphExec_t x = nullptr;
    const int ic = hip_ok(hipGraphInstantiate(&x, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (ic != JINF_HIP_OK) return ic;
    *out = x;
    return JINF_HIP_OK;
}

// The attention bound for steps whose lengths reach at most `len`.
int bound_for(int len, int max_ctx) {
    int b = 64;
    while (b < len) b *= 2;
    return b < max_ctx ? b : max_ctx;
}

// One token step on the engine's stream (the captured graph for the current
// bound, or the launches).
int step(jinf_hip_engine* e) {
    if (!e->use_graph) return enqueue_step(e);
    for (const auto& g : e->graphs)
        if (g.first == e->bound) return hip_ok(hipGraphLaunch(g.second, e->stream), "hipGraphLaunch");
    hipGraphExec_t x = nullptr;
    ENG_TRY(capture(e, &x));
    e->graphs.emplace_back(e->bound, x);
    return hip_ok(hipGraphLaunch(x, e->stream), "hipGraphLaunch");
}

int check_matrix(const void* p, int t, int rows, int cols, const char* what, int L) {
    if (!p || !is_matrix_type(t) || weight_bytes(t, rows, cols) == 0) {
        JINF_LOG("engine: layer %d %s: weight missing, type %d not served, or %d columns not "
                 "whole blocks", L, what, t, cols);
        return JINF_HIP_ERR_INVALID;
    }
    return JINF_HIP_OK;
}

int check_norm(const void* p, int t, const char* what, int L) {
    if (!p || !is_dense_type(t)) {
        JINF_LOG("engine: layer %d %s: norm weight missing or type %d not F32/F16", L, what, t);
        return JINF_HIP_ERR_INVALID;
    }
    return JINF_HIP_OK;
}

int validate(const jinf_hip_engine_desc* d) {
    if (d->n_layers < 0 || d->n_embd <= 0 || d->n_heads <= 0 || d->n_heads_kv <= 0 ||
        d->n_ff <= 0 || d->n_vocab <= 0 || d->max_context <= 0 ||
        (d->n_layers > 0 && !d->layers)) {
        JINF_LOG("engine: bad hyper-parameters");
        return JINF_HIP_ERR_INVALID;
    }
    if (d->n_embd % d->n_heads != 0 || d->n_heads % d->n_heads_kv != 0) {
        JINF_LOG("engine: n_embd %d / n_heads %d / n_heads_kv %d do not divide", d->n_embd,
                 d->n_heads, d->n_heads_kv);
        return JINF_HIP_ERR_INVALID;
    }
    const int hd = d->n_embd / d->n_heads;
    if (hd % 2 != 0 || hd > 512) {
        JINF_LOG("engine: head_dim %d must be even and at most 512", hd);
        return JINF_HIP_ERR_INVALID;
    }
    if (d->kv_type != JINF_HIP_F32 && d->kv_type != JINF_HIP_F16) return JINF_HIP_ERR_INVALID;
    if (!(d->rms_norm_eps >= 0.0f) || !(d->rope_freq_base > 0.0f)) return JINF_HIP_ERR_INVALID;
    const int kvd = d->n_heads_kv * hd;
    for (int L = 0; L < d->n_layers; ++L) {
        const jinf_hip_layer_weights& w = d->layers[L];
        ENG_TRY(check_norm(w.attn_norm, w.attn_norm_type, "attn_norm", L));
        ENG_TRY(check_norm(w.ffn_norm, w.ffn_norm_type, "ffn_norm", L));
        ENG_TRY(check_matrix(w.attn_q, w.attn_q_type, d->n_embd, d->n_embd, "attn_q", L));
        ENG_TRY(check_matrix(w.attn_k, w.attn_k_type, kvd, d->n_embd, "attn_k", L));
        ENG_TRY(check_matrix(w.attn_v, w.attn_v_type, kvd, d->n_embd, "attn_v", L));
        ENG_TRY(check_matrix(w.attn_output, w.attn_output_type, d->n_embd, d->n_embd,
                             "attn_output", L));
        ENG_TRY(check_matrix(w.ffn_gate, w.ffn_gate_type, d->n_ff, d->n_embd, "ffn_gate", L));
        ENG_TRY(check_matrix(w.ffn_up, w.ffn_up_type, d->n_ff, d->n_embd, "ffn_up", L));
        ENG_TRY(check_matrix(w.ffn_down, w.ffn_down_type, d->n_embd, d->n_ff, "ffn_down", L));
    }
    if (!d->token_embd || weight_bytes(d->token_embd_type, d->n_vocab, d->n_embd) == 0) {
        JINF_LOG("engine: token_embd missing or type %d not served", d->token_embd_type);
        return JINF_HIP_ERR_INVALID;
    }
    if (d->output_norm) ENG_TRY(check_norm(d->output_norm, d->output_norm_type, "output_norm", -1));
    if (d->output)
        ENG_TRY(check_matrix(d->output, d->output_type, d->n_vocab, d->n_embd, "output", -1));
    else
        ENG_TRY(check_matrix(d->token_embd, d->token_embd_type, d->n_vocab, d->n_embd,
                             "output (tied to token_embd)", -1));
    return JINF_HIP_OK;
}

void release(jinf_hip_engine* e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    for (const auto& g : e->graphs) (void)hipGraphExecDestroy(g.second);
    jinf_hip_batch_destroy(e->pre);  // before the cache it borrows
    if (e->h_tokens) (void)hipHostFree(e->h_tokens);
    if (e->kv) (void)hipFree(e->kv);
    if (e->act) (void)hipFree(e->act);
    if (e->owned_weights) (void)hipFree(e->owned_weights);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

int zero_state(jinf_hip_engine* e) {
    const size_t kv_total = e->kv_layer_bytes * 2 * (size_t)e->d.n_layers;
    if (kv_total) ENG_TRY(hip_ok(hipMemsetAsync(e->kv, 0, kv_total, e->stream), "hipMemsetAsync"));
    ENG_TRY(hip_ok(hipMemsetAsync(e->state, 0, kStateWords * 4, e->stream), "hipMemsetAsync"));
    ENG_TRY(hip_ok(hipMemsetAsync(e->tokens, 0, (size_t)e->d.max_context * 4, e->stream),
                   "hipMemsetAsync"));
    ENG_TRY(hip_ok(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
    e->n_past = 0;
    e->perf = jinf_hip_perf_stats{};
    return JINF_HIP_OK;
}

// Accumulates a call's host wall time and tokens into the engine's counters
// when it goes out of scope (src/engine.cpp:756-757 time the forward call).
struct PerfScope {
    jinf_hip_engine* e;
    int tokens = 0;
    std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
    explicit PerfScope(jinf_hip_engine* eng) : e(eng) {}
    ~PerfScope() {
        const std::chrono::duration<double, std::milli> dt = std::chrono::steady_clock::now() - t0;
        e->perf.total_ms += dt.count();
        e->perf.tokens_generated += tokens;
    }
};

int create(jinf_hip_engine** out, const jinf_hip_engine_desc* desc, void* owned) {
    jinf_hip_engine* e = new (std::nothrow) jinf_hip_engine();
    if (!e) return JINF_HIP_ERR_OOM;
    e->d = *desc;
    e->owned_weights = owned;
    e->layers.assign(desc->layers, desc->layers + desc->n_layers);
    e->d.layers = e->layers.data();
    if (!e->d.output) {
        e->d.output = e->d.token_embd;
        e->d.output_type = e->d.token_embd_type;
    }
    const jinf_hip_engine_desc& d = e->d;
    e->head_dim = d.n_embd / d.n_heads;
    e->q_dim = d.n_embd;
    e->kv_dim = d.n_heads_kv * e->head_dim;
    e->kv_es = d.kv_type == JINF_HIP_F16 ? 2 : 4;
    e->kv_layer_bytes = (size_t)d.max_context * e->kv_dim * e->kv_es;
    e->arg_parts = (d.n_vocab + 4 * kArgThreads - 1) / (4 * kArgThreads);
    if (e->arg_parts > kArgMaxParts) e->arg_parts = kArgMaxParts;
    if (d.kv_type == JINF_HIP_F16)
        e->ws_bytes = jinf_attention_workspace_bytes(1, d.n_heads, e->head_dim, d.max_context);

    // activation block layout
    size_t off = 0;
    auto take_f = [&](size_t count) {
        const size_t o = off;
        off = up_to(off + count * 4, kAlign);
        return o;
    };
    const size_t o_hidden = take_f(d.n_embd), o_q = take_f(e->q_dim);
    const size_t o_attn = take_f(e->q_dim);
    const size_t o_gate = take_f(d.n_ff), o_up = take_f(d.n_ff), o_logits = take_f(d.n_vocab);
    const size_t o_pv = take_f(kArgMaxParts), o_pi = take_f(kArgMaxParts);
    const size_t o_tok = take_f(d.max_context), o_state = take_f(kStateWords);
    const size_t o_ws = off;
    off = up_to(off + e->ws_bytes, kAlign);

    int rc = hip_ok(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking),
                    "hipStreamCreateWithFlags");
    if (rc == JINF_HIP_OK) rc = hip_ok(hipMalloc((void**)&e->act, off), "hipMalloc");
    const size_t kv_total = e->kv_layer_bytes * 2 * (size_t)d.n_layers;
    if (rc == JINF_HIP_OK && kv_total) rc = hip_ok(hipMalloc((void**)&e->kv, kv_total), "hipMalloc");
    if (rc == JINF_HIP_OK)
        rc = hip_ok(hipHostMalloc((void**)&e->h_tokens, ((size_t)d.max_context + 16) * 4,
                                  hipHostMallocDefault),
                    "hipHostMalloc");
    if (rc != JINF_HIP_OK) {
        release(e);
        return rc;
    }
    auto f = [&](size_t o) { return reinterpret_cast<float*>(e->act + o); };
    e->hidden = f(o_hidden);
    e->q = f(o_q);
    e->attn = f(o_attn);
    e->gate = f(o_gate);
    e->up = f(o_up);
    e->logits = f(o_logits);
    e->part_v = f(o_pv);
    e->part_i = reinterpret_cast<int32_t*>(e->act + o_pi);
    e->tokens = reinterpret_cast<int32_t*>(e->act + o_tok);
    e->state = reinterpret_cast<int32_t*>(e->act + o_state);
    e->ws = e->ws_bytes ? e->act + o_ws : nullptr;
    rc = hip_ok(hipMemsetAsync(e->act, 0, off, e->stream), "hipMemsetAsync");
    if (rc == JINF_HIP_OK) rc = zero_state(e);
    if (rc != JINF_HIP_OK) {
        release(e);
        return rc;
    }
    *out = e;
    return JINF_HIP_OK;
}

// ---- model files ----

// The layer tensors the forward loop reads, in the order the reference
// assigns them by name (src/engine.cpp:150-158).
constexpr const char* kLayerSlots[9] = {"attn_norm.weight", "ffn_norm.weight", "attn_q.weight",
                                        "attn_k.weight",    "attn_v.weight",   "attn_output.weight",
                                        "ffn_gate.weight",  "ffn_up.weight",   "ffn_down.weight"};

struct Want {
    std::string name;    // file tensor name (GGUF convention)
    int layer = -1;      // layer tensors: layer and slot in kLayerSlots
    int slot = -1;
    int64_t cols, rows;  // GGUF ne0, ne1 (rows 1 for a vector)
    bool matrix, optional;
    const void** ptr;
    int32_t* type;
    int64_t index = -1;
    size_t offset = 0;
};

// What the loader needs to know about one tensor of a model file.
struct FileTensor {
    int qtype;
    uint32_t n_dims;
    const int64_t* shape;
    uint64_t n_bytes;
};

// A model file: tensor lookup, description and upload.
struct ModelFile {
    std::function<int64_t(const Want&)> find;  // index or -1
    std::function<FileTensor(int64_t)> info;
    std::function<int(int64_t, void*, uint64_t, hipStream_t)> upload;
};

// Every tensor the forward loop reads is uploaded into one device allocation
// the engine owns (tensor starts 256-byte aligned), shapes and formats are
// checked, then the engine is created on them.
int create_from_file(jinf_hip_engine** out, jinf_hip_engine_desc d, const ModelFile& file,
                     int q4_0_ggml_order) {
    if (d.n_layers < 0 || d.n_embd <= 0 || d.n_heads <= 0 || d.n_heads_kv <= 0 ||
        d.n_embd % d.n_heads != 0) {
        JINF_LOG("engine: model hyper-parameters incomplete");
        return JINF_HIP_ERR_PARSE;
    }
    const int64_t n = d.n_embd, kvd = (int64_t)d.n_heads_kv * (d.n_embd / d.n_heads);
    std::vector<jinf_hip_layer_weights> layers((size_t)d.n_layers);
    std::vector<Want> want;
    auto add = [&](const std::string& name, int layer, int slot, int64_t cols, int64_t rows,
                   bool matrix, bool opt, const void** p, int32_t* t) {
        Want w;
        w.name = name;
        w.layer = layer;
        w.slot = slot;
        w.cols = cols;
        w.rows = rows;
        w.matrix = matrix;
        w.optional = opt;
        w.ptr = p;
        w.type = t;
        want.push_back(w);
    };
    add("token_embd.weight", -1, -1, n, d.n_vocab, true, false, &d.token_embd, &d.token_embd_type);
    for (int L = 0; L < d.n_layers; ++L) {
        jinf_hip_layer_weights& w = layers[L];
        const std::string b = "blk." + std::to_string(L) + ".";
        const void** ptrs[9] = {&w.attn_norm, &w.ffn_norm, &w.attn_q, &w.attn_k, &w.attn_v,
                                &w.attn_output, &w.ffn_gate, &w.ffn_up, &w.ffn_down};
        int32_t* types[9] = {&w.attn_norm_type, &w.ffn_norm_type, &w.attn_q_type,
                             &w.attn_k_type, &w.attn_v_type, &w.attn_output_type,
                             &w.ffn_gate_type, &w.ffn_up_type, &w.ffn_down_type};
        const int64_t cols[9] = {n, n, n, n, n, n, n, n, d.n_ff};
        const int64_t rows[9] = {1, 1, n, kvd, kvd, n, d.n_ff, d.n_ff, n};
        for (int k = 0; k < 9; ++k)
            add(b + kLayerSlots[k], L, k, cols[k], rows[k], k >= 2, false, ptrs[k], types[k]);
    }
    add("output_norm.weight", -1, -1, n, 1, false, true, &d.output_norm, &d.output_norm_type);
    add("output.weight", -1, -1, n, d.n_vocab, true, true, &d.output, &d.output_type);

    size_t total = 0;
    for (Want& w : want) {
        w.index = file.find(w);
        if (w.index < 0) {
            if (w.optional) continue;
            JINF_LOG("engine: tensor %s not in the file", w.name.c_str());
            return JINF_HIP_ERR_PARSE;
        }
        const FileTensor t = file.info(w.index);
        const int64_t rows = t.n_dims >= 2 ? t.shape[1] : 1;
        bool ok = t.shape[0] == w.cols && rows == w.rows && t.n_dims <= 2;
        ok = ok && (w.matrix ? (is_matrix_type(t.qtype) || is_dense_type(t.qtype))
                             : is_dense_type(t.qtype));
        ok = ok && weight_bytes(t.qtype, rows, t.shape[0]) == t.n_bytes;
        if (!ok) {
            JINF_LOG("engine: tensor %s: shape or type %d not usable", w.name.c_str(), t.qtype);
            return JINF_HIP_ERR_INVALID;
        }
        w.offset = total;
        total = up_to(total + t.n_bytes, kAlign);
        *w.type = t.qtype;
    }
    void* dev = nullptr;
    hipStream_t s = nullptr;
    int rc = hip_ok(hipMalloc(&dev, total ? total : kAlign), "hipMalloc");
    if (rc == JINF_HIP_OK)
        rc = hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    for (Want& w : want) {
        if (rc != JINF_HIP_OK) break;
        if (w.index < 0) continue;
        const FileTensor t = file.info(w.index);
        char* p = static_cast<char*>(dev) + w.offset;
        rc = file.upload(w.index, p, t.n_bytes, s);
        if (rc == JINF_HIP_OK && q4_0_ggml_order && t.qtype == kQ4_0)
            rc = jinf_hip_q4_0_repack_ggml(p, (int64_t)(t.n_bytes / 18), s);
        *w.ptr = p;
    }
    if (rc == JINF_HIP_OK) rc = hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (s) (void)hipStreamDestroy(s);
    d.layers = layers.data();
    if (rc == JINF_HIP_OK) rc = validate(&d);
    if (rc == JINF_HIP_OK) rc = create(out, &d, dev);
    else if (dev) (void)hipFree(dev);
    return rc;
}

}  // namespace

extern "C" int jinf_hip_engine_create(jinf_hip_engine** out, const jinf_hip_engine_desc* desc) {
    if (!out || !desc) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    ENG_TRY(validate(desc));
    return create(out, desc, nullptr);
}

extern "C" int jinf_hip_engine_create_gguf(jinf_hip_engine** out, const jinf_hip_gguf* file,
                                           int max_context, int kv_type, int q4_0_ggml_order) {
    if (!out || !file || max_context <= 0) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    const jinf_hip_gguf_hparams* hp = jinf_hip_gguf_hparams_of(file);
    if (!hp) return JINF_HIP_ERR_INVALID;
    jinf_hip_engine_desc d{};
    d.n_layers = (int)hp->n_layers;
    d.n_embd = (int)hp->n_embd;
    d.n_heads = (int)hp->n_heads;
    d.n_heads_kv = (int)hp->n_heads_kv;
    d.n_ff = (int)hp->n_ff;
    d.n_vocab = (int)hp->n_vocab;
    d.max_context = max_context;
    d.rms_norm_eps = hp->rms_norm_eps;
    d.rope_freq_base = hp->rope_freq_base;
    d.kv_type = kv_type;
    ModelFile f;
    f.find = [&](const Want& w) { return jinf_hip_gguf_find_tensor(file, w.name.c_str()); };
    f.info = [&](int64_t i) {
        const jinf_hip_gguf_tensor* t = jinf_hip_gguf_tensor_at(file, (uint64_t)i);
        return FileTensor{t->qtype, t->n_dims, t->shape, t->n_bytes};
    };
    f.upload = [&](int64_t i, void* dst, uint64_t bytes, hipStream_t s) {
        return jinf_hip_gguf_upload(file, (uint64_t)i, dst, bytes, s);
    };
    return create_from_file(out, d, f, q4_0_ggml_order);
}

extern "C" int jinf_hip_engine_create_nvmw(jinf_hip_engine** out, const jinf_hip_nvmw* file,
                                           int max_context, int kv_type) {
    if (!out || !file || max_context <= 0) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    const jinf_hip_nvmw_header* h = jinf_hip_nvmw_header_of(file);
    jinf_hip_engine_desc d{};
    d.n_layers = (int)h->n_layers;
    d.n_embd = (int)h->n_embd;
    d.n_heads = (int)h->n_heads;
    d.n_heads_kv = (int)h->n_heads_kv;
    d.n_ff = (int)h->n_ff;
    d.n_vocab = (int)h->n_vocab;
    d.max_context = max_context;
    d.rms_norm_eps = h->rms_norm_eps;
    d.rope_freq_base = h->rope_freq_base;
    d.kv_type = kv_type;
    // Layer tensors by layer index and name, the reference's rule
    // (src/engine.cpp:135-159): an entry of layer L whose name contains a
    // slot's suffix fills that slot (the first suffix that matches; a later
    // entry for the same slot replaces an earlier one).  The others by exact
    // name (src/engine.cpp:170-188).
    const int n_layers = d.n_layers > 0 ? d.n_layers : 0;
    std::vector<int64_t> slot((size_t)n_layers * 9, -1);
    const uint64_t nt = jinf_hip_nvmw_n_tensors(file);
    for (uint64_t i = 0; i < nt; ++i) {
        const jinf_hip_nvmw_tensor* t = jinf_hip_nvmw_tensor_at(file, i);
        if (t->layer_index < 0 || t->layer_index >= n_layers) continue;
        for (int k = 0; k < 9; ++k)
            if (strstr(t->name, kLayerSlots[k])) {
                slot[(size_t)t->layer_index * 9 + k] = (int64_t)i;
                break;
            }
    }
    ModelFile f;
    f.find = [&](const Want& w) -> int64_t {
        if (w.layer >= 0) return slot[(size_t)w.layer * 9 + w.slot];
        return jinf_hip_nvmw_find_tensor(file, w.name.c_str());
    };
    f.info = [&](int64_t i) {
        const jinf_hip_nvmw_tensor* t = jinf_hip_nvmw_tensor_at(file, (uint64_t)i);
        return FileTensor{t->qtype, t->n_dims, t->shape, t->n_bytes};
    };
    f.upload = [&](int64_t i, void* dst, uint64_t bytes, hipStream_t s) {
        return jinf_hip_nvmw_upload(file, (uint64_t)i, dst, bytes, s);
    };
    return create_from_file(out, d, f, 0);
}

extern "C" void jinf_hip_engine_destroy(jinf_hip_engine* e) { release(e); }

const jinf_hip_engine_desc* jinf::engine_desc(const jinf_hip_engine* e) { return e ? &e->d : nullptr; }

extern "C" int jinf_hip_engine_reset(jinf_hip_engine* e) {
    if (!e) return JINF_HIP_ERR_INVALID;
    return zero_state(e);
}

extern "C" int jinf_hip_engine_n_past(const jinf_hip_engine* e) { return e ? e->n_past : -1; }

extern "C" int jinf_hip_engine_use_graph(jinf_hip_engine* e, int on) {
    if (!e) return JINF_HIP_ERR_INVALID;
    e->use_graph = on != 0;
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_engine_forward(jinf_hip_engine* e, const int32_t* tokens, int n_tokens,
                                       const float** logits) {
    if (!e || !tokens || n_tokens <= 0 || !logits) return JINF_HIP_ERR_INVALID;
    const jinf_hip_engine_desc& d = e->d;
    if (n_tokens > d.max_context - e->n_past) {
        JINF_LOG("engine: %d tokens after %d exceed the context of %d", n_tokens, e->n_past,
                 d.max_context);
        return JINF_HIP_ERR_INVALID;
    }
    for (int t = 0; t < n_tokens; ++t)
        if (tokens[t] < 0 || tokens[t] >= d.n_vocab) {
            JINF_LOG("engine: token id %d outside [0, %d)", tokens[t], d.n_vocab);
            return JINF_HIP_ERR_INVALID;
        }
    // the tokens at positions n_past .. n_past + n_tokens - 1, and the end of
    // the provided tokens; both copies read pinned memory that is not touched
    // again before the stream is synchronized below
    memcpy(e->h_tokens, tokens, (size_t)n_tokens * 4);
    int32_t* fill_end = e->h_tokens + d.max_context;
    *fill_end = e->n_past + n_tokens;
    ENG_TRY(hip_ok(hipMemcpyAsync(e->tokens + e->n_past, e->h_tokens, (size_t)n_tokens * 4,
                                  hipMemcpyHostToDevice, e->stream),
                   "hipMemcpyAsync"));
    ENG_TRY(hip_ok(hipMemcpyAsync(e->state + kFillEnd, fill_end, 4, hipMemcpyHostToDevice,
                                  e->stream),
                   "hipMemcpyAsync"));
    e->bound = bound_for(e->n_past + n_tokens, d.max_context);
    PerfScope perf(e);
    int rc = JINF_HIP_OK;
    for (int t = 0; t < n_tokens && rc == JINF_HIP_OK; ++t) {
        rc = step(e);
        if (rc == JINF_HIP_OK) {
            ++e->n_past;
            ++perf.tokens;
        }
    }
    const int sc = hip_ok(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    if (rc != JINF_HIP_OK) return rc;
    if (sc != JINF_HIP_OK) return sc;
    *logits = e->logits;
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_engine_prefill(jinf_hip_engine* e, const int32_t* tokens, int n_tokens,
                                       const float** logits) {
    if (!e || !tokens || n_tokens <= 0 || !logits) return JINF_HIP_ERR_INVALID;
    const jinf_hip_engine_desc& d = e->d;
    if (e->pre_state == 0 && n_tokens > 1) {
        const int rc = batch_create_borrowed(&e->pre, e, kPrefillRows, e->kv, d.max_context,
                                             d.kv_type);
        if (rc != JINF_HIP_OK && rc != JINF_HIP_ERR_INVALID) return rc;
        e->pre_state = rc == JINF_HIP_OK ? 1 : -1;
    }
    if (n_tokens == 1 || !e->pre) return jinf_hip_engine_forward(e, tokens, n_tokens, logits);
    // the batch validates the ids and the context against position n_past
    batch_set_pos(e->pre, e->n_past);
    PerfScope perf(e);
    const float* lg = nullptr;
    ENG_TRY(jinf_hip_batch_prefill(e->pre, 0, tokens, n_tokens, &lg));
    // the prefill has finished (the call waits): bring the engine's tokens,
    // logits and state to where n_tokens forward steps leave them
    const int p0 = e->n_past, p1 = p0 + n_tokens;
    memcpy(e->h_tokens, tokens, (size_t)n_tokens * 4);
    ENG_TRY(hip_ok(hipMemcpyAsync(e->tokens + p0, e->h_tokens, (size_t)n_tokens * 4,
                                  hipMemcpyHostToDevice, e->stream),
                   "hipMemcpyAsync"));
    ENG_TRY(hip_ok(hipMemcpyAsync(e->logits, lg, (size_t)d.n_vocab * 4, hipMemcpyDeviceToDevice,
                                  e->stream),
                   "hipMemcpyAsync"));
    ENG_TRY(launch(eng_prefill_end_kernel, dim3(1), dim3(64), 0, e->stream, e->state, e->tokens,
                   batch_argmax(e->pre), p1, d.max_context));
    ENG_TRY(hip_ok(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
    e->n_past = p1;
    perf.tokens = n_tokens;
    *logits = e->logits;
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_engine_generate(jinf_hip_engine* e, const int32_t* prompt, int n_prompt,
                                        int32_t* output, int max_tokens, int* n_generated) {
    if (!e || !output || !n_generated) return JINF_HIP_ERR_INVALID;
    if (n_prompt > 0) {
        if (!prompt) return JINF_HIP_ERR_INVALID;
        const float* lg = nullptr;
        ENG_TRY(jinf_hip_engine_forward(e, prompt, n_prompt, &lg));
    } else if (e->n_past == 0) {
        return JINF_HIP_ERR_INVALID;
    }
    int32_t* best = e->h_tokens + e->d.max_context + 1;
    int generated = 0;
    e->bound = bound_for(e->n_past + (max_tokens > 0 ? max_tokens : 0), e->d.max_context);
    for (int i = 0; i < max_tokens; ++i) {
        // the argmax of the last step (already the token at position n_past)
        ENG_TRY(hip_ok(hipMemcpyAsync(best, e->state + kBest, 4, hipMemcpyDeviceToHost,
                                      e->stream),
                       "hipMemcpyAsync"));
        ENG_TRY(hip_ok(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
        output[generated++] = *best;
        if (*best == kEos) break;
        // feeding the token back would overrun the cache: stop, as the
        // reference does when its forward call fails (src/engine.cpp:800-801)
        if (e->n_past >= e->d.max_context) break;
        // the counters take each fed-back token's step up to its completion,
        // as the reference's forward call per token counts itself
        // (src/engine.cpp:753-757); the argmax read above stays outside
        PerfScope perf(e);
        if (step(e) != JINF_HIP_OK) break;
        if (hipStreamSynchronize(e->stream) != hipSuccess) break;
        ++e->n_past;
        perf.tokens = 1;
    }
    *n_generated = generated;
    return hip_ok(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
}

extern "C" int jinf_hip_engine_copy_logits(const jinf_hip_engine* e, float* dst, int n) {
    if (!e || !dst || n < 0 || n > e->d.n_vocab) return JINF_HIP_ERR_INVALID;
    if (n == 0) return JINF_HIP_OK;
    ENG_TRY(hip_ok(hipMemcpyAsync(dst, e->logits, (size_t)n * 4, hipMemcpyDefault, e->stream),
                   "hipMemcpyAsync"));
    return hip_ok(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
}

extern "C" const jinf_hip_perf_stats* jinf_hip_engine_get_stats(const jinf_hip_engine* e) {
    return e ? &e->perf : nullptr;
}

// ---- the reference's engine API by name (include/jinf/engine_api.h) ----

struct jinf_engine {
    jinf_hip_nvmw* file = nullptr;  // kept until destroy
    jinf_hip_engine* e = nullptr;
};

extern "C" int jinf_engine_create(jinf_engine** out, const jinf_engine_config* cfg) {
    if (!out) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    if (!cfg || !cfg->model_path || cfg->max_context <= 0) return JINF_HIP_ERR_INVALID;
    if (cfg->predictor_path) {
        JINF_LOG("engine: a sparse-FFN predictor (%s) is not supported", cfg->predictor_path);
        return JINF_HIP_ERR_INVALID;
    }
    jinf_engine* w = new (std::nothrow) jinf_engine();
    if (!w) return JINF_HIP_ERR_OOM;
    int rc = jinf_hip_nvmw_load(&w->file, cfg->model_path);
    if (rc == JINF_HIP_OK) rc = jinf_hip_engine_create_nvmw(&w->e, w->file, cfg->max_context, JINF_HIP_F32);
    if (rc != JINF_HIP_OK) {
        jinf_engine_destroy(w);
        return rc;
    }
    *out = w;
    return JINF_HIP_OK;
}

extern "C" void jinf_engine_destroy(jinf_engine* w) {
    if (!w) return;
    jinf_hip_engine_destroy(w->e);
    if (w->file) jinf_hip_nvmw_free(w->file);
    delete w;
}

extern "C" int jinf_engine_forward(jinf_engine* w, const int32_t* tokens, int n_tokens,
                                   float** logits) {
    if (!w || !logits) return JINF_HIP_ERR_INVALID;
    const float* lg = nullptr;
    const int rc = jinf_hip_engine_forward(w->e, tokens, n_tokens, &lg);
    if (rc == JINF_HIP_OK) *logits = const_cast<float*>(lg);
    return rc;
}

extern "C" int jinf_engine_generate(jinf_engine* w, const int32_t* prompt, int n_prompt,
                                    int32_t* output, int max_tokens, int* n_generated) {
    if (!w) return JINF_HIP_ERR_INVALID;
    return jinf_hip_engine_generate(w->e, prompt, n_prompt, output, max_tokens, n_generated);
}

extern "C" void jinf_engine_reset(jinf_engine* w) {
    if (w) (void)jinf_hip_engine_reset(w->e);
}

extern "C" const jinf_perf_stats* jinf_engine_get_stats(const jinf_engine* w) {
    return w ? jinf_hip_engine_get_stats(w->e) : nullptr;
}

extern "C" uint64_t jinf_hip_engine_step_weight_bytes(const jinf_hip_engine* e) {
    if (!e) return 0;
    const jinf_hip_engine_desc& d = e->d;
    const int64_t n = d.n_embd;
    uint64_t b = weight_bytes(d.token_embd_type, 1, n);
    for (const jinf_hip_layer_weights& w : e->layers) {
        b += weight_bytes(w.attn_norm_type, 1, n) + weight_bytes(w.ffn_norm_type, 1, n);
        b += weight_bytes(w.attn_q_type, e->q_dim, n);
        b += weight_bytes(w.attn_k_type, e->kv_dim, n) + weight_bytes(w.attn_v_type, e->kv_dim, n);
        b += weight_bytes(w.attn_output_type, n, e->q_dim);
        b += weight_bytes(w.ffn_gate_type, d.n_ff, n) + weight_bytes(w.ffn_up_type, d.n_ff, n);
        b += weight_bytes(w.ffn_down_type, n, d.n_ff);
    }
    if (d.output_norm) b += weight_bytes(d.output_norm_type, 1, n);
    b += weight_bytes(d.output_type, d.n_vocab, n);
    return b;
}
