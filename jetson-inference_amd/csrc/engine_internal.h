// Internal interface between the one-sequence engine and the batch decoder
// built on it (not exported in the public headers).
#pragma once

#include "jinf/engine_hip.h"

namespace jinf {

// The engine's model: device weights, hyper-parameters, output resolved
// (tied to token_embd when the model has none), layers valid while the
// engine exists.
const jinf_hip_engine_desc* engine_desc(const jinf_hip_engine* e);

// A batch over a borrowed cache kv of one sequence, laid out as the engine's
// ([n_layers] K caches, then [n_layers] V caches, max_context * kv_dim
// elements of kv_type each), for jinf_hip_batch_prefill(b, 0, ...) in chunks
// of `rows` tokens; its forward and generate calls are rejected.  kv is not
// freed by jinf_hip_batch_destroy.  Status 5 for a model the batched GEMVs
// do not take.
int batch_create_borrowed(jinf_hip_batch** out, const jinf_hip_engine* engine, int rows, void* kv,
                          int max_context, int kv_type);
// Sets the position of the borrowed sequence (its cache rows below pos are
// valid).
void batch_set_pos(jinf_hip_batch* b, int pos);
// Device word holding the borrowed sequence's last prefill argmax.
const int32_t* batch_argmax(const jinf_hip_batch* b);

// jinf_rmsnorm_qkv_rope (an RMSNorm weight required) for q and k of weight
// format qtype_qk and v of format qtype_v in one launch.  *launched false
// (status 0, nothing enqueued) when the shapes, alignments or format pair
// need one launch per format.
int rmsnorm_qkv_rope_two(const void* wq, const void* wk, int qtype_qk, const void* wv,
                         int qtype_v, const float* h, const void* norm_w, int norm_type,
                         float eps, int cols, float* q_out, void* k_cache, void* v_cache,
                         int kv_type, const int32_t* pos, int max_ctx, int head_dim,
                         int n_heads, int n_heads_kv, float freq_base, hipStream_t stream,
                         bool* launched);

}  // namespace jinf
