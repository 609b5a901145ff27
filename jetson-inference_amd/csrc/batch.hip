// Batched decode: n_seq sequences decoded together on one engine's weights,
// each with its own position and its own region of a batched KV cache
// [n_layers][n_seq][max_ctx][kv_dim].  One step decodes one token for every
// sequence that has one: the reference's per-token loop (src/engine.cpp:
// 684-760, per layer :418-511) with every GEMV run for all sequences at once
// on the matrix cores (jinf_*_batch), so each weight byte is read once per
// step instead of once per sequence.  Sequences without a token this step
// ("idle": id -1, or a full context) write nothing and keep their position.
//
// Device state: per sequence the position, the token decoded this step, the
// last argmax; a mode word selects where the step's tokens come from (the
// host's array, or each sequence's last argmax for greedy generation, which
// also records the emitted token in a history).  Every launch of a step reads
// positions and tokens from device memory, so the step is captured once as a
// HIP graph and replayed.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <new>
#include <vector>

#include "argmax_device.h"
#include "engine_internal.h"
#include "jinf_device.h"
#include "jinf_host.h"
#include "matvec_batch_internal.h"
#include "quant_device.h"

namespace jinf {
namespace {

constexpr int kBatEos = 2;  // end-of-sequence id (src/engine.cpp:796-797)
constexpr int kBatArgParts = 64;
enum { kMode = 0, kStep = 1, kStateWords = 64 };

// Tokens of this step: the host's (mode 0) or each sequence's last argmax
// (mode 1, recorded as emitted; end of sequence emitted and not decoded).  A
// sequence decodes when it has a token and room in its context.
__global__ void bat_begin_kernel(const int32_t* __restrict__ st, const int32_t* __restrict__ htok,
                                 const int32_t* __restrict__ cur, const int32_t* __restrict__ pos,
                                 int32_t* __restrict__ act, int32_t* __restrict__ positions,
                                 int32_t* __restrict__ lens, int32_t* __restrict__ hist,
                                 int hist_rows, int n_seq, int max_ctx) {
    const int s = blockIdx.x * 256 + threadIdx.x;
    if (s >= n_seq) return;
    int t;
    if (st[kMode] == 0) {
        t = htok[s];
    } else {
        t = cur[s];
        const int k = st[kStep];
        if (k < hist_rows) hist[(int64_t)k * n_seq + s] = t;
        if (t == kBatEos) t = -1;
    }
    const int p = pos[s];
    const bool a = t >= 0 && p < max_ctx;
    act[s] = a ? t : -1;
    positions[s] = a ? p : -1;
    lens[s] = a ? p + 1 : 0;
}

// Embedding rows of an F32 or F16 table; an idle sequence gets zeros.
template <typename T>
__global__ __launch_bounds__(256) void bat_embed_dense_kernel(float* __restrict__ out,
                                                              const T* __restrict__ table,
                                                              const int32_t* __restrict__ act,
                                                              int n_vocab, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int s = blockIdx.y;
    if (i >= n) return;
    const int id = act[s];
    float v = 0.0f;
    if (id >= 0 && id < n_vocab) {
        if constexpr (sizeof(T) == 2)
            v = h2f(table[(int64_t)id * n + i]);
        else
            v = table[(int64_t)id * n + i];
    }
    out[(int64_t)s * n + i] = v;
}

// Argmax part 1 per sequence (grid: parts x n_seq).
__global__ __launch_bounds__(kArgThreads) void bat_argmax_part_kernel(
    const float* __restrict__ logits, int n, float* __restrict__ pv, int* __restrict__ pi) {
    const float* x = logits + (int64_t)blockIdx.y * n;
    float bv = -INFINITY;
    int bi = n;
    for (int j = blockIdx.x * kArgThreads + threadIdx.x; j < n; j += gridDim.x * kArgThreads)
        take(bv, bi, x[j], j);
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.y * gridDim.x + blockIdx.x] = bv;
        pi[blockIdx.y * gridDim.x + blockIdx.x] = bi;
    }
}

// Argmax part 2 and the end of the step (one workgroup per sequence): the
// first index of the largest logit (NaN rules of src/engine.cpp:783-791); a
// sequence that decoded advances its position and its argmax becomes its
// next token; in mode 1 a sequence that did not decode has stopped.
__global__ __launch_bounds__(kArgThreads) void bat_argmax_end_kernel(
    const float* __restrict__ logits, int n, const float* __restrict__ pv,
    const int* __restrict__ pi, int parts, int32_t* __restrict__ st,
    const int32_t* __restrict__ act, int32_t* __restrict__ pos, int32_t* __restrict__ cur) {
    const int s = blockIdx.x;
    float bv = -INFINITY;
    int bi = n;
    for (int k = threadIdx.x; k < parts; k += kArgThreads) take(bv, bi, pv[s * parts + k], pi[s * parts + k]);
    block_best(bv, bi);
    if (threadIdx.x != 0) return;
    const float* x = logits + (int64_t)s * n;
    const int best = (__builtin_isnan(x[0]) || bi >= n) ? 0 : bi;
    if (act[s] >= 0) {
        pos[s] = pos[s] + 1;
        cur[s] = best;
    } else if (st[kMode] != 0) {
        cur[s] = -1;
    }
    // the last sequence's workgroup counts the step (mode 1 history row)
    if (s == gridDim.x - 1) st[kStep] = st[kStep] + 1;
}

// End of a prefill chunk (one workgroup): the argmax of the chunk's last
// token (same rules) becomes sequence seq's next token, and its position
// moves to new_pos.
__global__ __launch_bounds__(kArgThreads) void bat_prefill_end_kernel(
    const float* __restrict__ logits, int n, const float* __restrict__ pv,
    const int* __restrict__ pi, int parts, int32_t* __restrict__ pos,
    int32_t* __restrict__ cur, int new_pos) {
    float bv = -INFINITY;
    int bi = n;
    for (int k = threadIdx.x; k < parts; k += kArgThreads) take(bv, bi, pv[k], pi[k]);
    block_best(bv, bi);
    if (threadIdx.x != 0) return;
    *pos = new_pos;
    *cur = (__builtin_isnan(logits[0]) || bi >= n) ? 0 : bi;
}

size_t up256(size_t x) { return (x + 255) / 256 * 256; }

int hip_rc(hipError_t e, const char* what) {
    if (e == hipSuccess) return JINF_HIP_OK;
    JINF_LOG("batch: %s failed: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? JINF_HIP_ERR_OOM : JINF_HIP_ERR_DEVICE;
}

#define BAT_TRY(expr)                         \
    do {                                      \
        const int rc_ = (expr);               \
        if (rc_ != JINF_HIP_OK) return rc_;   \
    } while (0)

}  // namespace
}  // namespace jinf

using namespace jinf;

struct jinf_hip_batch {
    const jinf_hip_engine_desc* d = nullptr;
    int n_seq = 0, max_ctx = 0, kv_type = 0, kv_es = 4;
    int head_dim = 0, q_dim = 0, kv_dim = 0, arg_parts = 1, hist_rows = 0;
    char* act = nullptr;  // activations, state, workspaces
    char* kv = nullptr;   // K caches, then V caches
    bool kv_owned = true; // false: the engine's one-sequence cache, borrowed for its prefill
    size_t kv_layer_bytes = 0;
    float *hidden = nullptr, *q = nullptr, *attn = nullptr, *ff = nullptr, *up = nullptr;
    float* logits = nullptr;
    float* part_v = nullptr;
    int32_t *part_i = nullptr, *st = nullptr, *htok = nullptr, *cur = nullptr, *pos = nullptr;
    int32_t *acts = nullptr, *positions = nullptr, *lens = nullptr, *hist = nullptr;
    void* mws = nullptr;  // batched-GEMV workspace
    size_t mws_bytes = 0;
    float* dpart = nullptr;  // partial sums of the deferred split merges
    size_t dpart_bytes = 0;
    void* aws = nullptr;  // attention workspace
    size_t aws_bytes = 0;
    int32_t* h_io = nullptr;  // pinned: n_seq tokens, 16 words, 3 n_seq prefill row words
    std::vector<int> h_pos;   // host copy of the positions
    hipStream_t stream = nullptr;
    // captured steps, one per attention bound (a power of two >= 64, at most
    // max_ctx): the bound sets the attention's launch geometry and covers
    // every length the step can see
    std::vector<std::pair<int, hipGraphExec_t>> graphs;
    int bound = 0;
    bool use_graph = true;
};

namespace {

int bat_embed(jinf_hip_batch* b, int rows) {
    const jinf_hip_engine_desc& d = *b->d;
    const dim3 grid((d.n_embd + 255) / 256, rows);
    if (d.token_embd_type == JINF_HIP_F32)
        return launch(bat_embed_dense_kernel<float>, grid, dim3(256), 0, b->stream, b->hidden,
                      static_cast<const float*>(d.token_embd), b->acts, d.n_vocab, d.n_embd);
    if (d.token_embd_type == JINF_HIP_F16)
        return launch(bat_embed_dense_kernel<uint16_t>, grid, dim3(256), 0, b->stream, b->hidden,
                      static_cast<const uint16_t*>(d.token_embd), b->acts, d.n_vocab, d.n_embd);
    return jinf_dequant_rows(b->hidden, d.n_embd, d.token_embd, d.token_embd_type, d.n_vocab,
                             d.n_embd, b->acts, rows, JINF_HIP_F32, b->stream);
}

// `pend`: the previous layer's deferred down-projection residual add, merged
// into the residual stream by a launch ahead of the first GEMV's preparation.
// One GEMV launch per weight format of q, k and v (Q4_K_M: Q4_K q and k, Q6_K
// v), one epilogue launch for all of them.
int bat_qkv(jinf_hip_batch* b, const jinf_hip_layer_weights& w, void* kc, void* vc, int rows,
            int64_t ld_seq, MbDefer& pend) {
    const jinf_hip_engine_desc& d = *b->d;
    const void* W[3] = {w.attn_q, w.attn_k, w.attn_v};
    const int T[3] = {w.attn_q_type, w.attn_k_type, w.attn_v_type};
    BAT_TRY(rmsnorm_qkv_rope_batch_mixed(
        W, T, b->hidden, d.n_embd, w.attn_norm, w.attn_norm_type, d.rms_norm_eps, d.n_embd, b->q,
        b->q_dim, kc, vc, b->kv_type, ld_seq, b->positions, b->max_ctx, b->head_dim, d.n_heads,
        d.n_heads_kv, d.rope_freq_base, rows, b->mws, b->mws_bytes, &pend, b->dpart,
        b->dpart_bytes, b->stream));
    pend = MbDefer{};
    return JINF_HIP_OK;
}

// One step (src/engine.cpp:692-749 per row) over `rows` rows.  seq < 0: a
// decode step, row s = sequence s (every sequence; tokens and positions from
// the begin kernel).  seq >= 0: a prefill chunk, row i = prompt token i of
// sequence seq (tokens, positions and lengths already in the row arrays);
// the rows share the sequence's KV region (row stride 0), each writes its
// own position's K / V rows and attends up to them.
int bat_enqueue_rows(jinf_hip_batch* b, int rows, int seq, int new_pos) {
    const jinf_hip_engine_desc& d = *b->d;
    hipStream_t s = b->stream;
    const int n = d.n_embd, nff = d.n_ff, ns = rows;
    const float eps = d.rms_norm_eps;
    const bool prefill = seq >= 0;
    const int64_t ld_seq = prefill ? 0 : (int64_t)b->max_ctx * b->kv_dim;
    const size_t kv_off = prefill ? (size_t)seq * b->max_ctx * b->kv_dim * b->kv_es : 0;
    if (!prefill)
        BAT_TRY(launch(bat_begin_kernel, dim3((ns + 255) / 256), dim3(256), 0, s, b->st, b->htok,
                       b->cur, b->pos, b->acts, b->positions, b->lens, b->hist, b->hist_rows, ns,
                       b->max_ctx));
    BAT_TRY(bat_embed(b, ns));
    // The output and down projections' residual adds are deferred: their
    // column-split partial sums are added into the residual stream by a merge
    // launch ahead of the next GEMV's preparation, so the GEMVs need no
    // cross-workgroup merge (a counter with release / acquire ordering and a
    // merging workgroup per row group) of their own.
    MbDefer pend;
    for (int L = 0; L < d.n_layers; ++L) {
        const jinf_hip_layer_weights& w = d.layers[L];
        char* kc = b->kv + (size_t)L * b->kv_layer_bytes + kv_off;
        char* vc = b->kv + (size_t)(d.n_layers + L) * b->kv_layer_bytes + kv_off;
        BAT_TRY(bat_qkv(b, w, kc, vc, ns, ld_seq, pend));
        // the attention also writes the output projection's x records when
        // its work items are unsplit (short contexts), and that GEMV then
        // skips its preparation launch
        MbXRec xr;
        xr.rec = matvec_batch_add_xrec(b->mws, w.attn_output_type, n, b->q_dim, ns,
                                       &xr.chunk_cols);
        xr.mt = ns > 32 ? 2 : 1;
        BAT_TRY(attention_decode_xrec(b->attn, b->q_dim, b->q, b->q_dim, kc, vc, b->kv_type,
                                      b->kv_dim, ld_seq, b->lens, ns, b->bound, b->head_dim,
                                      d.n_heads, d.n_heads_kv, 0.0f, b->aws, b->aws_bytes, &xr,
                                      s));
        BAT_TRY(matvec_batch_add_defer(w.attn_output, w.attn_output_type, b->attn, b->q_dim, n,
                                       b->q_dim, ns, b->dpart, b->dpart_bytes, b->mws,
                                       b->mws_bytes, &pend, xr.wrote, s));
        if (w.ffn_gate_type == w.ffn_up_type) {
            BAT_TRY(rmsnorm_swiglu_matvec_batch_m(w.ffn_gate, w.ffn_up, w.ffn_gate_type, b->hidden,
                                                  n, w.ffn_norm, w.ffn_norm_type, eps, b->ff, nff,
                                                  nff, n, ns, b->mws, b->mws_bytes, &pend, s));
        } else {
            BAT_TRY(rmsnorm_matvec_batch_m(w.ffn_gate, w.ffn_gate_type, b->hidden, n, w.ffn_norm,
                                           w.ffn_norm_type, eps, b->ff, nff, nff, n, ns, b->mws,
                                           b->mws_bytes, &pend, s));
            BAT_TRY(rmsnorm_matvec_batch_m(w.ffn_up, w.ffn_up_type, b->hidden, n, w.ffn_norm,
                                           w.ffn_norm_type, eps, b->up, nff, nff, n, ns, b->mws,
                                           b->mws_bytes, nullptr, s));
            BAT_TRY(jinf_swiglu_rows(b->ff, nff, b->ff, nff, b->up, nff, ns, nff, JINF_HIP_F32, s));
        }
        pend = MbDefer{};
        BAT_TRY(matvec_batch_add_defer(w.ffn_down, w.ffn_down_type, b->ff, nff, n, nff, ns,
                                       b->dpart, b->dpart_bytes, b->mws, b->mws_bytes, &pend,
                                       false, s));
    }
    BAT_TRY(rmsnorm_matvec_batch_m(d.output, d.output_type, b->hidden, n, d.output_norm,
                                   d.output_norm_type, eps, b->logits, d.n_vocab, d.n_vocab, n, ns,
                                   b->mws, b->mws_bytes, &pend, s));
    if (prefill) {
        const float* last = b->logits + (int64_t)(ns - 1) * d.n_vocab;
        BAT_TRY(launch(bat_argmax_part_kernel, dim3(b->arg_parts, 1), dim3(kArgThreads), 0, s,
                       last, d.n_vocab, b->part_v, b->part_i));
        return launch(bat_prefill_end_kernel, dim3(1), dim3(kArgThreads), 0, s, last, d.n_vocab,
                      b->part_v, b->part_i, b->arg_parts, b->pos + seq, b->cur + seq, new_pos);
    }
    BAT_TRY(launch(bat_argmax_part_kernel, dim3(b->arg_parts, ns), dim3(kArgThreads), 0, s,
                   b->logits, d.n_vocab, b->part_v, b->part_i));
    return launch(bat_argmax_end_kernel, dim3(ns), dim3(kArgThreads), 0, s, b->logits, d.n_vocab,
                  b->part_v, b->part_i, b->arg_parts, b->st, b->acts, b->pos, b->cur);
}

int bat_enqueue_step(jinf_hip_batch* b) { return bat_enqueue_rows(b, b->n_seq, -1, 0); }

int bat_capture(jinf_hip_batch* b, hipGraphExec_t* out) {
    BAT_TRY(hip_rc(hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal),
                   "hipStreamBeginCapture"));
    const int rc = bat_enqueue_step(b);
    hipGraph_t g = nullptr;
    const int ec = hip_rc(hipStreamEndCapture(b->stream, &g), "hipStreamEndCapture");
    if (rc != JINF_HIP_OK || ec != JINF_HIP_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc != JINF_HIP_OK ? rc : ec;
    }
    hipGraphExec_t x = nullptr;
    const int ic = hip_rc(hipGraphInstantiate(&x, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (ic != JINF_HIP_OK) return ic;
    *out = x;
    return JINF_HIP_OK;
}

int bat_bound(const jinf_hip_batch* b, int len) {
    int v = 64;
    while (v < len) v *= 2;
    return v < b->max_ctx ? v : b->max_ctx;
}

int bat_max_pos(const jinf_hip_batch* b) {
    int m = 0;
    for (int p : b->h_pos) m = p > m ? p : m;
    return m;
}

int bat_step(jinf_hip_batch* b) {
    if (!b->use_graph) return bat_enqueue_step(b);
    for (const auto& g : b->graphs)
        if (g.first == b->bound) return hip_rc(hipGraphLaunch(g.second, b->stream), "hipGraphLaunch");
    hipGraphExec_t x = nullptr;
    BAT_TRY(bat_capture(b, &x));
    b->graphs.emplace_back(b->bound, x);
    return hip_rc(hipGraphLaunch(x, b->stream), "hipGraphLaunch");
}

void bat_release(jinf_hip_batch* b) {
    if (!b) return;
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    for (const auto& g : b->graphs) (void)hipGraphExecDestroy(g.second);
    if (b->h_io) (void)hipHostFree(b->h_io);
    if (b->kv && b->kv_owned) (void)hipFree(b->kv);
    if (b->act) (void)hipFree(b->act);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
}

// Clears the KV region and state of sequence `seq` (all when seq < 0).
int bat_reset(jinf_hip_batch* b, int seq) {
    const jinf_hip_engine_desc& d = *b->d;
    const size_t per_seq = (size_t)b->max_ctx * b->kv_dim * b->kv_es;
    for (int half = 0; half < 2 && b->kv_owned; ++half)
        for (int L = 0; L < d.n_layers; ++L) {
            char* base = b->kv + (size_t)(half * d.n_layers + L) * b->kv_layer_bytes;
            if (seq < 0)
                BAT_TRY(hip_rc(hipMemsetAsync(base, 0, b->kv_layer_bytes, b->stream), "hipMemsetAsync"));
            else
                BAT_TRY(hip_rc(hipMemsetAsync(base + (size_t)seq * per_seq, 0, per_seq, b->stream),
                               "hipMemsetAsync"));
        }
    const int lo = seq < 0 ? 0 : seq, cnt = seq < 0 ? b->n_seq : 1;
    BAT_TRY(hip_rc(hipMemsetAsync(b->pos + lo, 0, (size_t)cnt * 4, b->stream), "hipMemsetAsync"));
    BAT_TRY(hip_rc(hipMemsetAsync(b->cur + lo, 0xFF, (size_t)cnt * 4, b->stream), "hipMemsetAsync"));
    BAT_TRY(hip_rc(hipStreamSynchronize(b->stream), "hipStreamSynchronize"));
    for (int i = lo; i < lo + cnt; ++i) b->h_pos[i] = 0;
    return JINF_HIP_OK;
}

// Sets the mode word (and zeroes the step counter) from pinned memory.
int bat_set_mode(jinf_hip_batch* b, int mode) {
    int32_t* w = b->h_io + b->n_seq;
    w[0] = mode;
    w[1] = 0;
    return hip_rc(hipMemcpyAsync(b->st, w, 8, hipMemcpyHostToDevice, b->stream), "hipMemcpyAsync");
}

}  // namespace

namespace {

// kv_borrowed == nullptr: a batch with its own cache of n_seq regions.
// Otherwise the cache is kv_borrowed, one region (sequence 0) laid out as the
// engine's ([n_layers] K caches, then [n_layers] V caches, max_context *
// kv_dim elements each), and n_seq is the number of rows of a prefill chunk.
int bat_create(jinf_hip_batch** out, const jinf_hip_engine* engine, int n_seq, int max_context,
               int kv_type, void* kv_borrowed) {
    if (!out) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    const jinf_hip_engine_desc* dp = engine_desc(engine);
    if (!dp || n_seq < 1 || n_seq > 64 || max_context <= 0) return JINF_HIP_ERR_INVALID;
    if (kv_type != JINF_HIP_F32 && kv_type != JINF_HIP_F16) return JINF_HIP_ERR_INVALID;
    const jinf_hip_engine_desc& d = *dp;
    if (d.n_embd % 256 != 0 || d.n_ff % 256 != 0 || d.n_embd > 32768 || d.n_ff > 32768) {
        JINF_LOG("batch: n_embd %d and n_ff %d must be multiples of 256, at most 32768", d.n_embd,
                 d.n_ff);
        return JINF_HIP_ERR_INVALID;
    }
    jinf_hip_batch* b = new (std::nothrow) jinf_hip_batch();
    if (!b) return JINF_HIP_ERR_OOM;
    b->d = dp;
    b->n_seq = n_seq;
    b->max_ctx = max_context;
    b->kv_type = kv_type;
    b->kv_es = kv_type == JINF_HIP_F16 ? 2 : 4;
    b->head_dim = d.n_embd / d.n_heads;
    b->q_dim = d.n_embd;
    b->kv_dim = d.n_heads_kv * b->head_dim;
    b->kv_owned = kv_borrowed == nullptr;
    b->kv_layer_bytes = (size_t)(b->kv_owned ? n_seq : 1) * max_context * b->kv_dim * b->kv_es;
    b->arg_parts = (d.n_vocab + 4 * kArgThreads - 1) / (4 * kArgThreads);
    if (b->arg_parts > kBatArgParts) b->arg_parts = kBatArgParts;
    b->hist_rows = max_context < 256 ? max_context + 1 : 256;
    b->h_pos.assign(n_seq, 0);

    // workspace of the largest batched GEMV of a step
    const int n = d.n_embd, nff = d.n_ff;
    const int shapes[][2] = {{b->q_dim + 2 * b->kv_dim, n}, {n, b->q_dim}, {nff, n},
                             {n, nff},                      {d.n_vocab, n}};
    for (const auto& sh : shapes) {
        const size_t w = jinf_matvec_batch_workspace_bytes(sh[0], sh[1], n_seq);
        if (w > b->mws_bytes) b->mws_bytes = w;
    }
    b->aws_bytes = jinf_attention_workspace_bytes(n_seq, d.n_heads, b->head_dim, max_context);
    // partial sums of the deferred merges: output and down projections,
    // and the Q / K / V launch
    for (const auto& sh : {std::make_pair(n, b->q_dim), std::make_pair(n, nff)}) {
        const size_t w = matvec_batch_defer_bytes(sh.first, sh.second, n_seq);
        if (w > b->dpart_bytes) b->dpart_bytes = w;
    }
    // each layer's Q / K / V launches keep one partials region per format
    for (int L = 0; L < d.n_layers; ++L) {
        const jinf_hip_layer_weights& lw = d.layers[L];
        const int T[3] = {lw.attn_q_type, lw.attn_k_type, lw.attn_v_type};
        const size_t w = qkv_defer_bytes(T, b->q_dim, b->kv_dim, n, n_seq);
        if (w > b->dpart_bytes) b->dpart_bytes = w;
    }

    size_t off = 0;
    auto take_b = [&](size_t bytes) {
        const size_t o = off;
        off = up256(off + bytes);
        return o;
    };
    const size_t ns = (size_t)n_seq;
    const size_t o_hidden = take_b(ns * n * 4), o_q = take_b(ns * b->q_dim * 4);
    const size_t o_attn = take_b(ns * b->q_dim * 4), o_ff = take_b(ns * nff * 4);
    const size_t o_up = take_b(ns * nff * 4), o_logits = take_b(ns * d.n_vocab * 4);
    const size_t o_pv = take_b(ns * kBatArgParts * 4), o_pi = take_b(ns * kBatArgParts * 4);
    const size_t o_st = take_b(kStateWords * 4), o_htok = take_b(ns * 4), o_cur = take_b(ns * 4);
    const size_t o_pos = take_b(ns * 4), o_acts = take_b(ns * 4), o_positions = take_b(ns * 4);
    const size_t o_lens = take_b(ns * 4), o_hist = take_b((size_t)b->hist_rows * ns * 4);
    const size_t o_mws = take_b(b->mws_bytes), o_aws = take_b(b->aws_bytes);
    const size_t o_dpart = take_b(b->dpart_bytes);

    int rc = hip_rc(hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking), "hipStreamCreate");
    if (rc == JINF_HIP_OK) rc = hip_rc(hipMalloc((void**)&b->act, off), "hipMalloc");
    const size_t kv_total = b->kv_layer_bytes * 2 * (size_t)d.n_layers;
    if (!b->kv_owned)
        b->kv = static_cast<char*>(kv_borrowed);
    else if (rc == JINF_HIP_OK && kv_total)
        rc = hip_rc(hipMalloc((void**)&b->kv, kv_total), "hipMalloc");
    if (rc == JINF_HIP_OK)
        rc = hip_rc(hipHostMalloc((void**)&b->h_io, (4 * ns + 16) * 4, hipHostMallocDefault),
                    "hipHostMalloc");
    if (rc != JINF_HIP_OK) {
        bat_release(b);
        return rc;
    }
    auto f = [&](size_t o) { return reinterpret_cast<float*>(b->act + o); };
    auto i32 = [&](size_t o) { return reinterpret_cast<int32_t*>(b->act + o); };
    b->hidden = f(o_hidden);
    b->q = f(o_q);
    b->attn = f(o_attn);
    b->ff = f(o_ff);
    b->up = f(o_up);
    b->logits = f(o_logits);
    b->part_v = f(o_pv);
    b->part_i = i32(o_pi);
    b->st = i32(o_st);
    b->htok = i32(o_htok);
    b->cur = i32(o_cur);
    b->pos = i32(o_pos);
    b->acts = i32(o_acts);
    b->positions = i32(o_positions);
    b->lens = i32(o_lens);
    b->hist = i32(o_hist);
    b->mws = b->act + o_mws;
    b->dpart = f(o_dpart);
    b->aws = b->aws_bytes ? b->act + o_aws : nullptr;
    // zero everything (the workspaces' counters must start at zero)
    rc = hip_rc(hipMemsetAsync(b->act, 0, off, b->stream), "hipMemsetAsync");
    if (rc == JINF_HIP_OK) rc = bat_reset(b, -1);
    if (rc != JINF_HIP_OK) {
        bat_release(b);
        return rc;
    }
    *out = b;
    return JINF_HIP_OK;
}

}  // namespace

namespace jinf {

int batch_create_borrowed(jinf_hip_batch** out, const jinf_hip_engine* engine, int rows, void* kv,
                          int max_context, int kv_type) {
    if (!kv) return JINF_HIP_ERR_INVALID;
    return bat_create(out, engine, rows, max_context, kv_type, kv);
}

void batch_set_pos(jinf_hip_batch* b, int pos) { b->h_pos[0] = pos; }

const int32_t* batch_argmax(const jinf_hip_batch* b) { return b->cur; }

}  // namespace jinf

extern "C" int jinf_hip_batch_create(jinf_hip_batch** out, const jinf_hip_engine* engine, int n_seq,
                                     int max_context, int kv_type) {
    return bat_create(out, engine, n_seq, max_context, kv_type, nullptr);
}

extern "C" void jinf_hip_batch_destroy(jinf_hip_batch* b) { bat_release(b); }

extern "C" int jinf_hip_batch_reset(jinf_hip_batch* b, int seq) {
    if (!b || seq >= b->n_seq) return JINF_HIP_ERR_INVALID;
    return bat_reset(b, seq < 0 ? -1 : seq);
}

extern "C" int jinf_hip_batch_n_past(const jinf_hip_batch* b, int seq) {
    if (!b || seq < 0 || seq >= b->n_seq) return -1;
    return b->h_pos[seq];
}

extern "C" int jinf_hip_batch_use_graph(jinf_hip_batch* b, int on) {
    if (!b) return JINF_HIP_ERR_INVALID;
    b->use_graph = on != 0;
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_batch_forward(jinf_hip_batch* b, const int32_t* tokens,
                                      const float** logits) {
    // a borrowed cache holds one sequence: prefill only
    if (!b || !tokens || !logits || !b->kv_owned) return JINF_HIP_ERR_INVALID;
    const jinf_hip_engine_desc& d = *b->d;
    for (int s = 0; s < b->n_seq; ++s) {
        if (tokens[s] < -1 || tokens[s] >= d.n_vocab) {
            JINF_LOG("batch: token id %d outside [-1, %d)", tokens[s], d.n_vocab);
            return JINF_HIP_ERR_INVALID;
        }
        if (tokens[s] >= 0 && b->h_pos[s] >= b->max_ctx) {
            JINF_LOG("batch: sequence %d is at the end of its context (%d)", s, b->max_ctx);
            return JINF_HIP_ERR_INVALID;
        }
    }
    memcpy(b->h_io, tokens, (size_t)b->n_seq * 4);
    BAT_TRY(hip_rc(hipMemcpyAsync(b->htok, b->h_io, (size_t)b->n_seq * 4, hipMemcpyHostToDevice,
                                  b->stream),
                   "hipMemcpyAsync"));
    BAT_TRY(bat_set_mode(b, 0));
    b->bound = bat_bound(b, bat_max_pos(b) + 1);
    const int rc = bat_step(b);
    const int sc = hip_rc(hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc != JINF_HIP_OK) return rc;
    if (sc != JINF_HIP_OK) return sc;
    for (int s = 0; s < b->n_seq; ++s)
        if (tokens[s] >= 0) ++b->h_pos[s];
    *logits = b->logits;
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_batch_prefill(jinf_hip_batch* b, int seq, const int32_t* tokens,
                                      int n_tokens, const float** logits) {
    if (!b || seq < 0 || seq >= b->n_seq || n_tokens < 0 || (n_tokens > 0 && !tokens))
        return JINF_HIP_ERR_INVALID;
    const jinf_hip_engine_desc& d = *b->d;
    for (int i = 0; i < n_tokens; ++i)
        if (tokens[i] < 0 || tokens[i] >= d.n_vocab) {
            JINF_LOG("batch: token id %d outside [0, %d)", tokens[i], d.n_vocab);
            return JINF_HIP_ERR_INVALID;
        }
    const int p0 = b->h_pos[seq];
    if (n_tokens > b->max_ctx - p0) {
        JINF_LOG("batch: %d prompt tokens do not fit sequence %d's context (%d of %d used)",
                 n_tokens, seq, p0, b->max_ctx);
        return JINF_HIP_ERR_INVALID;
    }
    int32_t* rw = b->h_io + b->n_seq + 16;  // tokens, positions, lengths of a chunk
    int last = 0;
    for (int c = 0; c < n_tokens; c += b->n_seq) {
        const int m = n_tokens - c < b->n_seq ? n_tokens - c : b->n_seq;
        for (int i = 0; i < m; ++i) {
            rw[i] = tokens[c + i];
            rw[b->n_seq + i] = p0 + c + i;
            rw[2 * b->n_seq + i] = p0 + c + i + 1;
        }
        BAT_TRY(hip_rc(hipMemcpyAsync(b->acts, rw, (size_t)m * 4, hipMemcpyHostToDevice,
                                      b->stream), "hipMemcpyAsync"));
        BAT_TRY(hip_rc(hipMemcpyAsync(b->positions, rw + b->n_seq, (size_t)m * 4,
                                      hipMemcpyHostToDevice, b->stream), "hipMemcpyAsync"));
        BAT_TRY(hip_rc(hipMemcpyAsync(b->lens, rw + 2 * b->n_seq, (size_t)m * 4,
                                      hipMemcpyHostToDevice, b->stream), "hipMemcpyAsync"));
        b->bound = bat_bound(b, p0 + c + m);
        const int rc = bat_enqueue_rows(b, m, seq, p0 + c + m);
        // the pinned rows are rewritten for the next chunk: wait for this one
        const int sc = hip_rc(hipStreamSynchronize(b->stream), "hipStreamSynchronize");
        if (rc != JINF_HIP_OK) return rc;
        if (sc != JINF_HIP_OK) return sc;
        b->h_pos[seq] = p0 + c + m;
        last = m - 1;
    }
    if (logits) *logits = b->logits + (int64_t)last * d.n_vocab;
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_batch_generate(jinf_hip_batch* b, int32_t* output, int steps) {
    if (!b || !output || steps < 0 || !b->kv_owned) return JINF_HIP_ERR_INVALID;
    int rc = JINF_HIP_OK;
    // in chunks of the device history's rows
    for (int done = 0; done < steps && rc == JINF_HIP_OK;) {
        const int n = steps - done < b->hist_rows ? steps - done : b->hist_rows;
        rc = bat_set_mode(b, 1);
        b->bound = bat_bound(b, bat_max_pos(b) + n);
        for (int k = 0; k < n && rc == JINF_HIP_OK; ++k) rc = bat_step(b);
        if (rc == JINF_HIP_OK)
            rc = hip_rc(hipMemcpyAsync(output + (size_t)done * b->n_seq, b->hist,
                                       (size_t)n * b->n_seq * 4, hipMemcpyDefault, b->stream),
                        "hipMemcpyAsync");
        if (rc == JINF_HIP_OK)
            rc = hip_rc(hipMemcpyAsync(b->h_io, b->pos, (size_t)b->n_seq * 4,
                                       hipMemcpyDeviceToHost, b->stream),
                        "hipMemcpyAsync");
        if (rc == JINF_HIP_OK)
            rc = hip_rc(hipStreamSynchronize(b->stream), "hipStreamSynchronize");
        if (rc == JINF_HIP_OK)
            for (int s = 0; s < b->n_seq; ++s) b->h_pos[s] = b->h_io[s];
        done += n;
    }
    // refresh the host positions
    int32_t* hp = b->h_io;
    if (rc == JINF_HIP_OK)
        rc = hip_rc(hipMemcpyAsync(hp, b->pos, (size_t)b->n_seq * 4, hipMemcpyDeviceToHost,
                                   b->stream),
                    "hipMemcpyAsync");
    const int sc = hip_rc(hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc != JINF_HIP_OK) return rc;
    if (sc != JINF_HIP_OK) return sc;
    for (int s = 0; s < b->n_seq; ++s) b->h_pos[s] = hp[s];
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_batch_copy_logits(const jinf_hip_batch* b, float* dst) {
    if (!b || !dst) return JINF_HIP_ERR_INVALID;
    BAT_TRY(hip_rc(hipMemcpyAsync(dst, b->logits, (size_t)b->n_seq * b->d->n_vocab * 4,
                                  hipMemcpyDefault, b->stream),
                   "hipMemcpyAsync"));
    return hip_rc(hipStreamSynchronize(b->stream), "hipStreamSynchronize");
}
