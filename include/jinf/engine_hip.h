/*
 * jinf MI355X: the decode engine -- the reference's per-token forward loop
 * (src/engine.cpp:418-511 per layer, :684-760 per token) running entirely on
 * this library's kernels, with every weight resident in device memory.
 *
 * One token step is: embedding gather; per layer RMSNorm (fused with the
 * previous residual add), q/k/v dequant-GEMVs, RoPE at position n_past, the
 * K/V rows written into the layer's cache at n_past, GQA attention over
 * n_past + 1 positions, output GEMV, residual add fused into the FFN RMSNorm,
 * gate/up GEMVs, SiLU * up, down GEMV; final residual add + RMSNorm, output
 * GEMV to the logits, and an on-device greedy argmax.  Positions and lengths
 * live in device memory, so the whole step is captured once as a HIP graph
 * and replayed for every token.
 *
 * Status codes are jinf_status values (0 OK, 1 I/O, 2 parse, 3 device,
 * 4 out of memory, 5 invalid argument).  An engine is used by one host
 * thread at a time.  This header includes no HIP or CUDA header.
 */
#ifndef JINF_ENGINE_HIP_H
#define JINF_ENGINE_HIP_H

#include <stdint.h>
#include "gguf_hip.h"
#include "kernels_ext.h"
#include "nvmw_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct jinf_hip_engine jinf_hip_engine;

/* Device pointers and jinf_qtype codes of one layer's weights, the fields of
 * jinf_layer_ptrs (include/jinf/engine.h:56-81).  Norm weights are F32 (0)
 * or F16 (1); matrices are Q4_0 (2), Q8_0 (8), Q4_K (12) or Q6_K (14),
 * [rows = outputs, cols = inputs] in blocks along the inputs. */
typedef struct jinf_hip_layer_weights {
    const void* attn_norm;
    const void* ffn_norm;
    const void* attn_q;
    const void* attn_k;
    const void* attn_v;
    const void* attn_output;
    const void* ffn_gate;
    const void* ffn_up;
    const void* ffn_down;
    int32_t attn_norm_type;
    int32_t ffn_norm_type;
    int32_t attn_q_type;
    int32_t attn_k_type;
    int32_t attn_v_type;
    int32_t attn_output_type;
    int32_t ffn_gate_type;
    int32_t ffn_up_type;
    int32_t ffn_down_type;
} jinf_hip_layer_weights;

/* A model whose weights already sit in device memory (owned by the caller,
 * who keeps them alive while the engine exists).  token_embd: F32, F16, Q4_0,
 * Q8_0, Q4_K or Q6_K rows of n_embd; output: a matrix type (NULL: tied to
 * token_embd).  kv_type: JINF_HIP_F32 (the reference's cache) or JINF_HIP_F16
 * (attention on the matrix cores). */
typedef struct jinf_hip_engine_desc {
    int   n_layers, n_embd, n_heads, n_heads_kv, n_ff, n_vocab, max_context;
    float rms_norm_eps, rope_freq_base;
    int   kv_type;
    const void* token_embd;
    int32_t     token_embd_type;
    const void* output_norm;
    int32_t     output_norm_type;
    const void* output;
    int32_t     output_type;
    const jinf_hip_layer_weights* layers;   /* n_layers entries */
} jinf_hip_engine_desc;

/* Creates the engine: KV caches [n_layers][max_context][n_heads_kv * head_dim]
 * (zeroed), activation buffers and its own stream (replaces jinf_engine_create,
 * src/engine.cpp:40-220, for a resident model). */
int jinf_hip_engine_create(jinf_hip_engine** out, const jinf_hip_engine_desc* desc);

/* Same from a GGUF file: every tensor the forward loop reads (token_embd,
 * blk.N.{attn_norm,attn_q,attn_k,attn_v,attn_output,ffn_norm,ffn_gate,ffn_up,
 * ffn_down}, output_norm, output -- tied to token_embd when absent) is
 * uploaded into one device allocation the engine owns; hyper-parameters come
 * from the file.  q4_0_ggml_order != 0 converts Q4_0 tensors written in
 * upstream ggml's element order to jinf's (jinf_hip_q4_0_repack_ggml). */
int jinf_hip_engine_create_gguf(jinf_hip_engine** out, const jinf_hip_gguf* file,
                                int max_context, int kv_type, int q4_0_ggml_order);

/* Same from a .nvmw file (the reference engine's model format,
 * jinf_engine_create src/engine.cpp:40-188): hyper-parameters from its
 * header; every tensor, hot or cold, is uploaded (the whole model stays
 * resident, so the reference's NVMe streaming of cold layers has no
 * counterpart); layer tensors are matched by layer index and name suffix as
 * the reference does, token_embd / output_norm / output by exact name
 * (output absent: tied to token_embd).  A neuron-bundle index is ignored:
 * the FFN is decoded dense. */
int jinf_hip_engine_create_nvmw(jinf_hip_engine** out, const jinf_hip_nvmw* file,
                                int max_context, int kv_type);

void jinf_hip_engine_destroy(jinf_hip_engine* e);

/* Zeroes the KV caches and n_past (jinf_engine_reset, src/engine.cpp:294-302). */
int jinf_hip_engine_reset(jinf_hip_engine* e);

int jinf_hip_engine_n_past(const jinf_hip_engine* e);

/* Decodes n_tokens tokens one at a time (jinf_engine_forward,
 * src/engine.cpp:684-760); *logits receives the device pointer of the last
 * token's n_vocab fp32 logits (valid until the next call).  Returns after the
 * work has finished.  Status 5 when the context would exceed max_context or
 * a token id is outside [0, n_vocab). */
int jinf_hip_engine_forward(jinf_hip_engine* e, const int32_t* tokens, int n_tokens,
                            const float** logits);

/* Decodes a prompt of n_tokens tokens in steps of up to 64 tokens, every GEMV
 * running on a step's tokens at once on the matrix cores (the batched path
 * of jinf_hip_batch_prefill, over this engine's own cache) and token i
 * attending to the positions up to its own.  Leaves the engine where
 * jinf_hip_engine_forward on the same tokens would (position advanced by
 * n_tokens, next token the last token's argmax, *logits the last token's
 * logits); per token the arithmetic is that loop's, with the batched GEMVs'
 * rounding (within the same tolerances of the oracle, not bit-equal to
 * forward).  One token, or a model whose n_embd or n_ff is not a multiple
 * of 256 or above 32768, goes through jinf_hip_engine_forward.  Same status
 * codes as forward.  The reference feeds a prompt one token at a time
 * (src/engine.cpp:684-760); this entry point has no counterpart there. */
int jinf_hip_engine_prefill(jinf_hip_engine* e, const int32_t* tokens, int n_tokens,
                            const float** logits);

/* Greedy generation (jinf_engine_generate, src/engine.cpp:762-805): the
 * prompt (if any) is decoded, then up to max_tokens argmax tokens (first
 * maximum on ties) are emitted and fed back; token 2 (end of sequence) is
 * emitted and stops generation.  The prompt goes through
 * jinf_hip_engine_forward (one token at a time); for a long prompt, call
 * jinf_hip_engine_prefill first and then generate with n_prompt 0. */
int jinf_hip_engine_generate(jinf_hip_engine* e, const int32_t* prompt, int n_prompt,
                             int32_t* output, int max_tokens, int* n_generated);

/* Copies the first n (<= n_vocab) logits of the last decoded token to dst
 * (host or device memory) and waits for the copy; the reference's caller
 * reads them through the device pointer forward returns. */
int jinf_hip_engine_copy_logits(const jinf_hip_engine* e, float* dst, int n);

/* 1 (default): replay the captured token step as a HIP graph; 0: launch the
 * kernels one by one (same results). */
int jinf_hip_engine_use_graph(jinf_hip_engine* e, int on);

/* Bytes of weights one token step reads (every matrix once, one embedding
 * row, the norms): the numerator of the decode bandwidth. */
uint64_t jinf_hip_engine_step_weight_bytes(const jinf_hip_engine* e);

/* Performance counters, the reference's jinf_perf_stats
 * (include/jinf/engine.h:14-22) field for field: total_ms is the host wall
 * time spent running tokens through the model (each forward / prefill call,
 * and in generate each fed-back token's step up to its completion, as the
 * reference's generate counts only its forward calls; the argmax reads
 * between steps are not counted), tokens_generated the tokens run through
 * the model (prompt and fed-back tokens, as the reference's forward counts
 * them, src/engine.cpp:756-757).  The streaming and per-phase fields stay zero, as
 * the reference leaves them on its resident path.  Reset clears them. */
typedef struct jinf_hip_perf_stats {
    double total_ms;
    double nvme_read_ms;
    double gpu_compute_ms;
    double attention_ms;
    double ffn_ms;
    int tokens_generated;
    double nvme_bytes_read;
} jinf_hip_perf_stats;

/* The engine's counters (replaces jinf_engine_get_stats,
 * include/jinf/engine.h:175-176; NULL for a NULL engine). */
const jinf_hip_perf_stats* jinf_hip_engine_get_stats(const jinf_hip_engine* e);

/* ---- Batched decode: n_seq (1..64) sequences decoded together on one
 * engine's weights (the engine must outlive the batch).  Each sequence has
 * its own position and its own region of a batched KV cache
 * [n_layers][n_seq][max_context][n_heads_kv * head_dim] of kv_type; one step
 * decodes one token for every sequence that has one, with every GEMV run for
 * all of them at once on the matrix cores (jinf_*_batch), so each weight
 * byte is read once per step.  The reference has no counterpart: it decodes
 * one sequence (src/engine.cpp:684-805); per sequence the arithmetic is that
 * loop's.  Needs n_embd and n_ff multiples of 256, at most 32768. ---- */
typedef struct jinf_hip_batch jinf_hip_batch;

int  jinf_hip_batch_create(jinf_hip_batch** out, const jinf_hip_engine* engine, int n_seq,
                           int max_context, int kv_type);
void jinf_hip_batch_destroy(jinf_hip_batch* b);

/* Clears sequence seq's KV region and position (every sequence when seq < 0). */
int  jinf_hip_batch_reset(jinf_hip_batch* b, int seq);
int  jinf_hip_batch_n_past(const jinf_hip_batch* b, int seq);

/* One step: tokens[s] (n_seq ids, -1 = sequence s idle this step) decoded at
 * each sequence's position; *logits receives the device pointer of the
 * [n_seq][n_vocab] fp32 logits (an idle sequence's row is unspecified).
 * Returns after the work has finished.  Status 5 for an id outside
 * [-1, n_vocab) or a token for a sequence whose context is full. */
int  jinf_hip_batch_forward(jinf_hip_batch* b, const int32_t* tokens, const float** logits);

/* Prompt of sequence seq: decodes its n_tokens ids (each in [0, n_vocab))
 * in chunks of up to n_seq tokens per step, every GEMV running on a chunk's
 * tokens at once and token i attending to the sequence's positions up to its
 * own, so the sequence ends where n_tokens forward steps of its own would
 * leave it (position advanced by n_tokens, next token the last token's
 * argmax); other sequences are untouched.  The last chunk's per-token logits
 * occupy rows 0 .. m - 1 of the batch's logits (the last token's at row
 * (n_tokens - 1) mod n_seq); *logits (may be NULL) receives the device
 * pointer of that row.  Status 5 when the prompt does not fit the sequence's
 * context or an id is outside [0, n_vocab).  The reference feeds a prompt
 * one token at a time (src/engine.cpp:684-760); per token the arithmetic is
 * that loop's. */
int  jinf_hip_batch_prefill(jinf_hip_batch* b, int seq, const int32_t* tokens, int n_tokens,
                            const float** logits);

/* Greedy generation for `steps` steps (jinf_hip_engine_generate per
 * sequence): at each step every sequence emits its last argmax (the one
 * computed by the previous forward or generate step) into output[step *
 * n_seq + s] and decodes it; a sequence that emits token 2 (end of
 * sequence), has no token, or has a full context stops and emits -1 from
 * then on. */
int  jinf_hip_batch_generate(jinf_hip_batch* b, int32_t* output, int steps);

/* Copies the last step's [n_seq][n_vocab] logits to dst (host or device). */
int  jinf_hip_batch_copy_logits(const jinf_hip_batch* b, float* dst);

/* 1 (default): replay the captured step as a HIP graph; 0: launch eagerly. */
int  jinf_hip_batch_use_graph(jinf_hip_batch* b, int on);

#ifdef __cplusplus
}
#endif

#endif /* JINF_ENGINE_HIP_H */
