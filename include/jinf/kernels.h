/*
 * jinf MI355X kernels: drop-in C-ABI entry points.
 *
 * These are the per-layer elementwise/reduction launchers that jinf's engine
 * declares in its own extern "C" block (reference src/engine.cpp:12-31) and
 * calls per token (src/engine.cpp:418-511, 684-760).  Names and parameter
 * lists are kept identical so engine.cpp links against libjinf_hip.so with no
 * source change other than cudaStream_t -> hipStream_t (both are opaque
 * pointer-sized stream handles).
 *
 * Contract (same as the reference launchers):
 *   - every pointer is a DEVICE pointer owned by the caller;
 *   - work is enqueued asynchronously on `stream`; nothing here allocates,
 *     frees or synchronizes; no mutable global state, so concurrent calls on
 *     different streams are safe;
 *   - functions return void; n <= 0 (or zero heads) is a no-op instead of an
 *     invalid launch.  Arguments that the kernels cannot serve (see each
 *     function) print one line to stderr and enqueue nothing, mirroring the
 *     reference's stderr report for an unsupported qtype
 *     (cuda/matmul_kernels.cu:221-223).
 *
 * This header includes no HIP or CUDA header.
 */
#ifndef JINF_KERNELS_H
#define JINF_KERNELS_H

/* Same opaque handle type as <hip/hip_runtime_api.h>; redeclaring an
 * identical typedef is legal in C11 and C++. */
typedef struct ihipStream_t* hipStream_t;

#ifdef __cplusplus
extern "C" {
#endif

/* y[i] = (x[i] * r) * w[i], r = 1/sqrt(sum(x^2)/n + eps), one fp32 row of n.
 * weight_type: 0 = fp32 weight, 1 = fp16 weight, anything else = fp32
 * (as cuda/rmsnorm_kernel.cu:79-83).  output == input is allowed (the engine's
 * final norm runs in place, src/engine.cpp:737-741).
 * Replaces jinf_cuda_rmsnorm, cuda/rmsnorm_kernel.cu:65-85. */
void jinf_cuda_rmsnorm(float* output, const float* input, const void* weight,
                       int n, float eps, int weight_type, hipStream_t stream);

/* In-place interleaved RoPE of one token at position `pos`: for every q head,
 * then every k head, pair (2i, 2i+1) is rotated by pos * base^(-2i/head_dim).
 * head_dim must be even and <= 512.
 * Replaces jinf_cuda_rope, cuda/rope_kernel.cu:54-61. */
void jinf_cuda_rope(float* q, float* k, int head_dim, int n_heads, int n_heads_kv,
                    int pos, float freq_base, hipStream_t stream);

/* output[i] = (gate[i] / (1 + exp(-gate[i]))) * up[i]; output may alias gate
 * or up (the engine runs it with output == gate, src/engine.cpp:502).
 * Replaces jinf_cuda_silu_mul, cuda/silu_kernel.cu:22-27. */
void jinf_cuda_silu_mul(float* output, const float* gate, const float* up,
                        int n, hipStream_t stream);

/* One fp32 row: y = exp(x - max x) / sum exp(x - max x); output may alias input.
 * Each output within 1e-5 relative of the exact softmax (results below 1e-30
 * within 1e-30 absolutely).
 * Replaces jinf_cuda_softmax, cuda/softmax_kernel.cu:46-51. */
void jinf_cuda_softmax(float* output, const float* input, int n, hipStream_t stream);

/* a[i] += b[i], fp32, in place.
 * Replaces jinf_cuda_residual_add, cuda/matmul_kernels.cu:227-231. */
void jinf_cuda_residual_add(float* a, const float* b, int n, hipStream_t stream);

/* Dequantize n_blocks consecutive GGUF Q4_0 blocks (18 bytes: fp16 scale d,
 * then 16 bytes of nibbles) to 32*n_blocks floats in jinf's interleaved order:
 * out[32b+2j] = ((qs[j] & 15) - 8) * d, out[32b+2j+1] = ((qs[j] >> 4) - 8) * d.
 * `data` may have any byte alignment.
 * Replaces jinf_cuda_dequantize_q4_0, cuda/dequant_kernels.cu:116-122. */
void jinf_cuda_dequantize_q4_0(const void* data, float* output, int n_blocks,
                               hipStream_t stream);

/* Dequantize n_blocks consecutive Q4_K super-blocks (144 bytes, 256 values:
 * d, dmin, 12 packed 6-bit scale/min bytes in the reference's own packing,
 * 128 bytes of nibbles) to fp32, bit-identical to the reference.
 * Replaces jinf_cuda_dequantize_q4_K, cuda/dequant_kernels.cu:124-129. */
void jinf_cuda_dequantize_q4_K(const void* data, float* output, int n_blocks,
                               hipStream_t stream);

/* Dequantize n_blocks consecutive Q8_0 blocks (34 bytes: d, 32 int8).
 * Replaces jinf_cuda_dequantize_q8_0, cuda/dequant_kernels.cu:131-137. */
void jinf_cuda_dequantize_q8_0(const void* data, float* output, int n_blocks,
                               hipStream_t stream);

/* Dequantize n_blocks consecutive Q6_K super-blocks (210 bytes: ql[128],
 * qh[64], int8 scales[16], d) to fp32, bit-identical to the reference.
 * Replaces jinf_cuda_dequantize_q6_K, cuda/dequant_kernels.cu:139-146. */
void jinf_cuda_dequantize_q6_K(const void* data, float* output, int n_blocks,
                               hipStream_t stream);

/* y[row] = sum_j W[row, j] * x[j] for a [rows, cols] matrix stored as GGUF
 * blocks along the columns, fp32 x and y (4-byte aligned).  qtype 2 (Q4_0),
 * 8 (Q8_0), 12 (Q4_K) and 14 (Q6_K) are served, as in the reference, with its
 * element orders and dequantized weights; cols must be a multiple of the
 * block size (32, or 256 for the K formats).  Any other qtype prints one
 * stderr line and enqueues nothing.
 * Replaces jinf_cuda_dequant_matvec, cuda/matmul_kernels.cu:198-225 (kernels
 * :8-185). */
void jinf_cuda_dequant_matvec(const void* weight, const float* input, float* output,
                              int rows, int cols, int qtype, hipStream_t stream);

/* GQA decode attention for one query token: for every query head h (kv head
 * h / (n_heads / n_heads_kv)), out_h = softmax_t((q_h . k_t) / sqrt(head_dim))
 * applied to v_t over t < n_past, all fp32.  k_cache and v_cache are one
 * layer's [max_ctx][n_heads_kv][head_dim] fp32 caches (the engine writes the
 * current token's rows at position n_past - 1 first, src/engine.cpp:446-453).
 * n_past <= 0 enqueues nothing (output untouched); n_past > max_ctx prints one
 * stderr line and enqueues nothing (the reference would read past the cache).
 * head_dim <= 1024.  Nothing is allocated: the interface has no workspace.
 * Replaces jinf_cuda_attention, cuda/attention_kernel.cu:100-115 (kernel
 * :25-96). */
void jinf_cuda_attention(float* output, const float* q, const float* k_cache,
                         const float* v_cache, int head_dim, int n_heads,
                         int n_heads_kv, int n_past, int max_ctx, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JINF_KERNELS_H */
