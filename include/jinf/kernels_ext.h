/*
 * jinf MI355X kernels: batched / fp16 / fused entry points.
 *
 * The reference launchers (kernels.h) take one fp32 token row per call.  These
 * entry points run the same arithmetic over many rows per launch, in fp16 or
 * fp32 storage, and fuse the residual add into RMSNorm.  They have no
 * one-to-one counterpart in the reference; each names the reference code
 * whose semantics it batches.
 *
 * Common rules:
 *   - pointers are DEVICE pointers; all work is asynchronous on `stream`;
 *     nothing allocates, frees or synchronizes; no mutable global state;
 *   - `ld_*` arguments are row strides in ELEMENTS of the storage type;
 *   - fp16 tensors are IEEE binary16 stored as uint16_t; arithmetic is fp32
 *     with one round-to-nearest-even to fp16 per stored value;
 *   - return JINF_HIP_OK, JINF_HIP_ERR_INVALID (bad argument, nothing
 *     enqueued) or JINF_HIP_ERR_DEVICE (the launch failed).  The values equal
 *     jinf_status JINF_OK / JINF_ERR_CUDA / JINF_ERR_INVALID
 *     (reference include/jinf/common.h:9-16);
 *   - zero rows / zero columns is JINF_HIP_OK with nothing enqueued.
 *
 * This header includes no HIP or CUDA header.
 */
#ifndef JINF_KERNELS_EXT_H
#define JINF_KERNELS_EXT_H

#include <stdint.h>
#include "kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

enum jinf_hip_status {
    JINF_HIP_OK = 0,
    JINF_HIP_ERR_IO = 1,
    JINF_HIP_ERR_PARSE = 2,
    JINF_HIP_ERR_DEVICE = 3,
    JINF_HIP_ERR_OOM = 4,
    JINF_HIP_ERR_INVALID = 5
};

/* Storage types; codes equal jinf_qtype F32/F16 (reference include/jinf/quant.h:8-11). */
enum jinf_hip_dtype {
    JINF_HIP_F32 = 0,
    JINF_HIP_F16 = 1
};

/* Library version string and the gfx target it was built for. */
const char* jinf_hip_version(void);

/* Per-row RMSNorm: out[r,i] = (x[r,i] * rs_r) * w[i],
 * rs_r = 1/sqrt(sum_i x[r,i]^2 / n + eps).  act_type selects fp32/fp16
 * storage of in/out; weight_type 0 = fp32, 1 = fp16.  out may alias in.
 * Semantics of cuda/rmsnorm_kernel.cu:9-61, batched over rows. */
int jinf_rmsnorm_rows(void* out, int ld_out, const void* in, int ld_in,
                      const void* weight, int n_rows, int n, float eps,
                      int act_type, int weight_type, hipStream_t stream);

/* Fused residual add + RMSNorm, one HBM pass:
 *   residual[r,i] = residual[r,i] + delta[r,i]   (stored, rounded to act_type)
 *   out[r,i]      = rmsnorm(residual[r,:])[i] * w[i]
 * The norm consumes the rounded stored residual, exactly like the reference's
 * separate residual_add then rmsnorm launches (src/engine.cpp:466->487,
 * 508->429).  out may alias delta (not residual). */
int jinf_residual_rmsnorm_rows(void* out, int ld_out, void* residual, int ld_res,
                               const void* delta, int ld_delta, const void* weight,
                               int n_rows, int n, float eps, int act_type,
                               int weight_type, hipStream_t stream);

/* In-place interleaved RoPE over n_tokens tokens.  q is [n_tokens, ld_q] with
 * n_heads*head_dim live elements per token, k is [n_tokens, ld_k] with
 * n_heads_kv*head_dim.  Token t uses positions[t], or pos0 + t when
 * positions is NULL.  head_dim even, <= 512.  Semantics of
 * cuda/rope_kernel.cu:8-50 applied per token. */
int jinf_rope_rows(void* q, int ld_q, void* k, int ld_k, const int32_t* positions,
                   int pos0, int n_tokens, int head_dim, int n_heads, int n_heads_kv,
                   float freq_base, int act_type, hipStream_t stream);

/* SwiGLU: out[r,i] = silu(gate[r,i]) * up[r,i], silu(g) = g / (1 + exp(-g)).
 * out may alias gate or up.  Semantics of cuda/silu_kernel.cu:6-18, batched. */
int jinf_swiglu_rows(void* out, int ld_out, const void* gate, int ld_gate,
                     const void* up, int ld_up, int n_rows, int n, int act_type,
                     hipStream_t stream);

/* Residual add a[r,i] += b[r,i] (rounded to act_type).
 * Semantics of cuda/matmul_kernels.cu:189-194, batched. */
int jinf_residual_add_rows(void* a, int ld_a, const void* b, int ld_b, int n_rows,
                           int n, int act_type, hipStream_t stream);

/* Masked fp32 row softmax.  Row r has live length
 *   L_r = lens ? clamp(lens[r / rows_per_len], 0, n_cols) : n_cols
 * and out[r, j] = exp(s_j - m) / sum_k exp(s_k - m) for j < L_r, with
 * s_j = scale * in[r, j] and m = max_j s_j.  Elements j >= L_r are neither
 * read nor written; L_r == 0 leaves the row untouched.  out may alias in.
 * rows_per_len (> 0) lets all query heads of one sequence share one length
 * entry; lens then holds ceil(n_rows / rows_per_len) values.  scale must be
 * finite and > 0 (1 for pre-scaled scores).
 * Semantics of cuda/softmax_kernel.cu:8-42 and the attention softmax phase
 * cuda/attention_kernel.cu:59-87 (length n_past = pos + 1).  Accuracy: each
 * exponential within 6.5e-6 relative for every normal fp32 result, each
 * output within 1e-5 relative of the exact softmax (results below 1e-30 within
 * 1e-30 absolutely). */
int jinf_softmax_rows_f32(float* out, int ld_out, const float* in, int ld_in,
                          int n_rows, int n_cols, const int32_t* lens,
                          int rows_per_len, float scale, hipStream_t stream);

/* GGUF Q4_0 token-embedding gather + dequant.  table holds n_vocab rows of
 * n_embd/32 blocks (18 bytes each, any byte alignment); output row i
 * (ld_out elements apart) is the dequantized table row ids[i], or table row i
 * when ids is NULL.  An id outside [0, n_vocab) yields a row of +0.0 (the
 * reference does not check ids, src/engine.cpp:311-312).  out_type fp32 or
 * fp16; fp16 values are one RNE rounding of the exact fp32 product, so the
 * result is bit-exact.  n_embd % 32 == 0.  Semantics of
 * src/engine.cpp:311-317 + cuda/dequant_kernels.cu:6-21 + src/quant.cpp:49-60. */
int jinf_embed_q4_0(void* out, int ld_out, const void* table, int n_vocab,
                    int n_embd, const int32_t* ids, int n_ids, int out_type,
                    hipStream_t stream);

/* GGUF block codes (values of jinf_qtype, reference include/jinf/quant.h:8-24)
 * served by jinf_matvec, jinf_dequant_rows and jinf_cuda_dequant_matvec. */
enum jinf_hip_qtype {
    JINF_HIP_Q4_0 = 2,
    JINF_HIP_Q8_0 = 8,
    JINF_HIP_Q4_K = 12,
    JINF_HIP_Q6_K = 14
};

/* Dequant-GEMV y = W x with a status return: W [rows, cols] stored as qtype
 * blocks along the columns (any byte alignment), x and y fp32 (4-byte
 * aligned); cols a multiple of the block size (32 or 256).  Same arithmetic as
 * jinf_cuda_dequant_matvec.  Fast path: W and x 16-byte aligned, cols a
 * multiple of 256 (2048 for Q6_K) and at most 28672.  Semantics of
 * cuda/matmul_kernels.cu:8-185. */
int jinf_matvec(const void* weight, int qtype, const float* x, float* y, int rows, int cols,
                hipStream_t stream);

/* jinf_matvec with qtype = JINF_HIP_Q4_0. */
int jinf_matvec_q4_0(const void* weight, const float* x, float* y, int rows, int cols,
                     hipStream_t stream);

/* ---- Dequant-GEMVs fused with the launches around them in the reference's
 * per-layer sequence (src/engine.cpp:418-511, :736-747).  Same weights and
 * formats as jinf_matvec; each result equals the unfused sequence's up to the
 * fp32 rounding of the dot products.  Vectors are fp32, 4-byte aligned; the
 * fast path wants weights, h/x and g 16-byte aligned, cols a multiple of 256
 * (2048 for Q6_K) and at most 28672, any other shape runs a slower generic
 * kernel.  No output may overlap another argument (jinf_matvec_add's y is
 * its own addend). ---- */

/* y = W x^ with x^_j = fl32(fl32(h_j * rs) * g_j), rs = 1/sqrt(sum h^2 / cols
 * + eps) (the RMSNorm of jinf_rmsnorm_rows, computed inside the GEMV):
 * the attention / FFN / final RMSNorm and the GEMV that reads its output
 * (src/engine.cpp:429+432, :487+489, :738+744).  norm_w NULL: x^ = h (plain
 * GEMV).  norm_type: 0 fp32, 1 fp16 weights g. */
int jinf_rmsnorm_matvec(const void* weight, int qtype, const float* h, const void* norm_w,
                        int norm_type, float eps, float* y, int rows, int cols,
                        hipStream_t stream);

/* y[r] = y[r] + (W x)[r]: a projection and the residual add that follows it
 * (output projection + residual, src/engine.cpp:461-466; down + residual,
 * :504-508). */
int jinf_matvec_add(const void* weight, int qtype, const float* x, float* y, int rows,
                    int cols, hipStream_t stream);

/* out[i] = silu(g_i) * u_i with g = W_gate x^, u = W_up x^ (x^ as in
 * jinf_rmsnorm_matvec; SiLU as jinf_cuda_silu_mul): the FFN RMSNorm, gate and
 * up GEMVs and SiLU * up of src/engine.cpp:487-502 in one launch; only the
 * n_ff products are written.  Both matrices [n_ff, cols] of qtype. */
int jinf_rmsnorm_swiglu_matvec(const void* w_gate, const void* w_up, int qtype, const float* h,
                               const void* norm_w, int norm_type, float eps, float* out,
                               int n_ff, int cols, hipStream_t stream);

/* Attention input side of one token at position *pos (device int32)
 * (src/engine.cpp:429-453): with x^ as in jinf_rmsnorm_matvec,
 *   q_out           = RoPE(W_q x^)       [n_heads * head_dim]
 *   k_cache row pos = RoPE(W_k x^)       [n_heads_kv * head_dim]
 *   v_cache row pos = W_v x^
 * RoPE as jinf_rope_rows at position *pos; the cache rows are
 * k_cache/v_cache + pos * n_heads_kv * head_dim elements of kv_type (F32, or
 * F16 rounded once); *pos outside [0, max_ctx) skips the cache stores.  A
 * NULL weight skips its projection; the others share qtype and cols.
 * head_dim even, <= 512. */
int jinf_rmsnorm_qkv_rope(const void* w_q, const void* w_k, const void* w_v, int qtype,
                          const float* h, const void* norm_w, int norm_type, float eps, int cols,
                          float* q_out, void* k_cache, void* v_cache, int kv_type,
                          const int32_t* pos, int max_ctx, int head_dim, int n_heads,
                          int n_heads_kv, float freq_base, hipStream_t stream);

/* ---- Batched dequant-GEMVs on the matrix cores: the per-token products of
 * src/engine.cpp:429-508 for n_batch (1..64) sequences decoded together, so
 * that each weight byte read serves all of them.  Row b of x / h / y is
 * ld_x / ld_h / ld_y elements after row b - 1.  Same weights and formats as
 * jinf_matvec with cols a multiple of 256 and at most 32768 and every matrix
 * 16-byte aligned (the bytes up to the next 16-byte boundary past a matrix's
 * end are read, as any device allocation allows; other shapes return 5), x / h
 * 16-byte aligned with ld a multiple of 4.  Products are exact fp16 x fp16 on
 * the matrix cores with x split into two fp16 halves under a power-of-two
 * scale per sequence (about 22 significant bits); each result equals the fp32
 * dot product up to the fp32 rounding of the sums.
 *
 * RMSNorm variants: x^ = fl32(fl32(h * rs) * g) exactly as jinf_rmsnorm_rows
 * computes it (norm_w NULL: x^ = h); norm_type 0 fp32, 1 fp16.
 *
 * Workspace (required): jinf_matvec_batch_workspace_bytes(rows, cols,
 * n_batch) bytes, 256-byte aligned and zero-filled before its first use.  It
 * holds x prepared for the matrix cores and, for launches that split the
 * columns over several workgroups, their partial sums and counters (the
 * counters return to zero at the end of every call, so the workspace is
 * reused without clearing, also across graph replays).  One workspace must
 * not be used by two calls that may run at the same time. ---- */

size_t jinf_matvec_batch_workspace_bytes(int rows, int cols, int n_batch);

/* y[b] = W x[b]. */
int jinf_matvec_batch(const void* weight, int qtype, const float* x, int ld_x, float* y,
                      int ld_y, int rows, int cols, int n_batch, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* y[b] += W x[b] (output projection / down projection + residual add,
 * src/engine.cpp:461-466, :504-508). */
int jinf_matvec_batch_add(const void* weight, int qtype, const float* x, int ld_x, float* y,
                          int ld_y, int rows, int cols, int n_batch, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* y[b] = W x^[b]: RMSNorm + GEMV (src/engine.cpp:738+744). */
int jinf_rmsnorm_matvec_batch(const void* weight, int qtype, const float* h, int ld_h,
                              const void* norm_w, int norm_type, float eps, float* y, int ld_y,
                              int rows, int cols, int n_batch, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* y[b][i] = silu((W_gate x^[b])_i) * (W_up x^[b])_i (src/engine.cpp:487-502);
 * i < n_ff. */
int jinf_rmsnorm_swiglu_matvec_batch(const void* w_gate, const void* w_up, int qtype,
                                     const float* h, int ld_h, const void* norm_w, int norm_type,
                                     float eps, float* y, int ld_y, int n_ff, int cols,
                                     int n_batch, void* workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/* jinf_rmsnorm_qkv_rope for n_batch sequences: sequence b's q row goes to
 * q + b * ld_q, its K / V rows to k_cache / v_cache + b * ld_seq +
 * positions[b] * n_heads_kv * head_dim (elements of kv_type), RoPE at
 * positions[b]; a position outside [0, max_ctx) skips that sequence's cache
 * stores.  ld_seq is at least max_ctx * n_heads_kv * head_dim, or 0: every
 * row then writes into the same cache (the tokens of one prompt; their
 * positions must differ).  cols = n_embd. */
int jinf_rmsnorm_qkv_rope_batch(const void* w_q, const void* w_k, const void* w_v, int qtype,
                                const float* h, int ld_h, const void* norm_w, int norm_type,
                                float eps, int cols, float* q, int ld_q, void* k_cache,
                                void* v_cache, int kv_type, int64_t ld_seq,
                                const int32_t* positions, int max_ctx, int head_dim, int n_heads,
                                int n_heads_kv, float freq_base, int n_batch, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* Gather + dequant of table rows for any qtype above (the engine's embedding
 * dispatch by table type, src/engine.cpp:311-334): output row i (ld_out
 * elements apart) is table row ids[i] (row i when ids is NULL), n_embd values
 * from n_embd / block_size blocks; an id outside [0, n_vocab) gives +0.0.
 * Weights are bit-identical to the reference's dequantizers
 * (cuda/dequant_kernels.cu:6-110); fp16 output is one RNE rounding of them.
 * Q4_0 runs jinf_embed_q4_0. */
int jinf_dequant_rows(void* out, int ld_out, const void* table, int qtype, int n_vocab,
                      int n_embd, const int32_t* ids, int n_ids, int out_type,
                      hipStream_t stream);

/* Batched GQA decode attention (cuda/attention_kernel.cu:25-96 over many
 * sequences, with an fp16 or fp32 KV cache): for sequence s and query head h
 * (kv head h / (n_heads / n_heads_kv)),
 *   out[s, h*hd:(h+1)*hd] = sum_t softmax_t(scale * q[s,h] . k[s,t,kv]) v[s,t,kv]
 * over t < lens[s] (clamped to [0, max_ctx]); a sequence with no position
 * gets zeros.  q and out are fp32 with row strides ld_q, ld_out (elements).
 * Cache element (s, t, kv head j, dim d) is at s*ld_seq + t*ld_pos + j*hd + d
 * in k_cache / v_cache, of kv_type JINF_HIP_F32 or JINF_HIP_F16; ld_seq is at
 * least max_ctx * ld_pos when n_seq > 1, or 0 (every row reads the same
 * cache: the tokens of one prompt, each with its own length).
 * scale = 0 means 1/sqrt(head_dim); otherwise finite and > 0.  lens is a
 * device array of n_seq int32.  Fast path: head_dim 64 or 128, caches, q
 * and strides 16-byte aligned; an fp16 cache then runs on the matrix cores
 * (|q * scale| < 65504).  Nothing is allocated.  workspace (device memory,
 * optional: NULL or too small runs every sequence in one work item) lets an
 * fp16-cache call split long contexts (chunks of at least 256 positions)
 * over several workgroups, which merge their partial results themselves; it
 * needs jinf_attention_workspace_bytes(n_seq, n_heads, head_dim, max_ctx)
 * bytes, zero-filled before its first use (every call leaves its merge
 * counters at zero again, so it is reused without clearing), and must not be
 * shared by calls running concurrently. */
int jinf_attention_decode(float* out, int ld_out, const float* q, int ld_q,
                          const void* k_cache, const void* v_cache, int kv_type,
                          int64_t ld_pos, int64_t ld_seq, const int32_t* lens,
                          int n_seq, int max_ctx, int head_dim, int n_heads,
                          int n_heads_kv, float scale, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes jinf_attention_decode can use to split long contexts
 * (0 for an empty shape). */
size_t jinf_attention_workspace_bytes(int n_seq, int n_heads, int head_dim, int max_ctx);

/* jinf_attention_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments, results and kernels as jinf_attention_decode with a workspace
 * (bit-identical outputs); the split contexts keep their merge counters and
 * chunk records in a library-owned scratch array in device memory instead:
 * 16 KiB of counters plus 8 MiB of records, one copy per device, held until
 * the process ends.  Nothing is allocated or freed by the call.
 *   - The first call on a device looks the scratch up (hipGetSymbolAddress)
 *     with that device current; make each call with the stream's device
 *     current.  A caller that captures the call in a graph makes one call on
 *     the device before capturing (a call with n_seq 0 does the lookup and
 *     enqueues nothing); the captured call then records only kernel nodes
 *     (its counters are cleared by a kernel, not a memset node).
 *   - A shape whose split would need more than the scratch holds (records of
 *     n_seq * n_heads * chunks * (head_dim + 2) floats above 8 MiB, e.g.
 *     127 sequences x 64 heads over 8192 positions) runs its contexts
 *     unsplit, as jinf_attention_decode does with too small a workspace, and
 *     gives that call's bits.
 *   - Every call on one device shares that device's scratch (each clears the
 *     counters it uses first): calls that may run at the same time on one
 *     device, on different streams, race and must not be issued. */
int jinf_attention_decode_noalloc(float* out, int ld_out, const float* q, int ld_q,
                                  const void* k_cache, const void* v_cache, int kv_type,
                                  int64_t ld_pos, int64_t ld_seq, const int32_t* lens,
                                  int n_seq, int max_ctx, int head_dim, int n_heads,
                                  int n_heads_kv, float scale, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JINF_KERNELS_EXT_H */
