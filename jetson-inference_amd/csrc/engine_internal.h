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

}  // namespace jinf
