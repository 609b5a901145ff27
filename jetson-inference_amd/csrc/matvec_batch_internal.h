// Internal interface of the batched GEMVs for the batch decoder (not in the
// public headers): a residual add whose column-split partial sums are left
// for the next normed GEMV call to merge (a launch of its own ahead of that
// call's preparation), instead of being merged by the GEMV's last workgroup
// of each row group.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>

namespace jinf {

// ---- prepared x records (the batched GEMVs' matrix-core operand) ----
//
// One record per 256-column slab: [MT M-tiles][16 k-steps][hi, lo][64 lanes]
// 16-byte fragments, lane (token % 32) + 32 h holding columns 16 t + 8 h ..
// + 7 of k-step t in the order (0, 4, 1, 5, 2, 6, 3, 7); then inv_s[32 MT]
// (1 / s per token) and Q4_K's sums of the scaled x over each 32-column
// sub-block, [8][32 MT].
__host__ __device__ constexpr int mb_rec_bytes(int mt) { return mt * 32768 + 2048 * mt; }

// Exponent ex of the power-of-two scale s = 2^(15 - ex) that puts the largest
// magnitude m in [2^14, 2^15) (15 for zero or non-finite m, at least -100).
__device__ __forceinline__ int mb_scale_exp(float m) {
    int ex = 15;
    if (m > 0.0f && m <= 3.4e38f) {
        (void)frexpf(m, &ex);  // m < 2^ex
        ex = ex < -100 ? -100 : ex;
    }
    return ex;
}

// The 8 columns of group gi (slab columns 8 gi .. 8 gi + 7) of token b into
// the slab's record r as fp16 hi = fp16(v s), lo = fp16(v s - hi); returns
// the sum of the scaled values (for the Q4_K sub-block sums).
__device__ __forceinline__ float mb_put_group(uint8_t* r, int b, int gi, const float (&v)[8],
                                              float sc) {
    const int t = gi >> 1, h = gi & 1;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // fragment slots 2 i, 2 i + 1 hold columns i and 4 + i of the group
        const float a0 = v[i] * sc, a1 = v[4 + i] * sc;
        const _Float16 h0 = (_Float16)a0, h1 = (_Float16)a1;
        const _Float16 l0 = (_Float16)(a0 - (float)h0), l1 = (_Float16)(a1 - (float)h1);
        hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
    }
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += v[e] * sc;
    uint8_t* f = r + (((b >> 5) * 16 + t) * 2) * 1024 + ((b & 31) + 32 * h) * 16;
    *reinterpret_cast<uint4*>(f) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *reinterpret_cast<uint4*>(f + 1024) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    return sum;
}

// The slab data of group gi: sum32 (the sum over the group's 32-column
// sub-block) from the first group of each sub-block, 1 / s from group 0.
__device__ __forceinline__ void mb_put_meta(uint8_t* r, int mt, int b, int gi, float sum32,
                                            int ex) {
    float* meta = reinterpret_cast<float*>(r + mt * 32768);
    if ((gi & 3) == 0) meta[32 * mt + (gi >> 2) * 32 * mt + b] = sum32;
    if (gi == 0) meta[b] = ldexpf(1.0f, ex - 15);
}

// Records written by the launch that produces the output projection's input
// (the attention, at short contexts): rec is that GEMV's record area, whose
// per-split scales cover chunk_cols columns each; the producer sets wrote
// when it wrote every record, and the GEMV then skips its preparation.
struct MbXRec {
    uint8_t* rec = nullptr;
    int mt = 1;
    int chunk_cols = 0;
    bool wrote = false;
};

// The record area and per-split chunk width (0: the input is not prepared per
// split) of matvec_batch_add_defer at this shape and workspace.
uint8_t* matvec_batch_add_xrec(void* workspace, int qtype, int rows, int cols, int n_batch,
                               int* chunk_cols);

// jinf_attention_decode (include/jinf/kernels_ext.h) that also writes the
// output projection's x records into xr when it can (xr->wrote): every work
// item unsplit, the fp16 matrix-core kernel, one work item's query-head
// columns equal to xr->chunk_cols.
int attention_decode_xrec(float* out, int ld_out, const float* q, int ld_q, const void* k_cache,
                          const void* v_cache, int kv_type, int64_t ld_pos, int64_t ld_seq,
                          const int32_t* lens, int n_seq, int max_ctx, int head_dim, int n_heads,
                          int n_heads_kv, float scale, void* workspace, size_t workspace_bytes,
                          MbXRec* xr, hipStream_t stream);

// Partial sums of a deferred residual add y += W x: part[s][b][r] for split
// s < k, sequence b < n_batch, row r < rows (stride elements between splits);
// ss / mx: room for the merge's statistics of the new rows, per 2048-row
// slice (sum of squares, largest |y g| for the normed GEMV that follows).
struct MbDefer {
    float* part = nullptr;
    int k = 0;
    int64_t stride = 0;
    double* ss = nullptr;
    float* mx = nullptr;
};

// Bytes of the partial sums of matvec_batch_add_defer at this shape.
size_t matvec_batch_defer_bytes(int rows, int cols, int n_batch);

// jinf_matvec_batch_add's products (x_ready: x already prepared in the
// workspace's records, see MbXRec), with the residual add left pending in
// *out (part: matvec_batch_defer_bytes bytes, 16-byte aligned).  y is not
// touched: the next call below that takes `pend` with h = y first adds the
// partial sums into h (summed in split order, as the GEMV's own merge does),
// then normalizes.
int matvec_batch_add_defer(const void* weight, int qtype, const float* x, int ld_x, int rows,
                           int cols, int n_batch, float* part, size_t part_bytes, void* workspace,
                           size_t workspace_bytes, MbDefer* out, bool x_ready, hipStream_t stream);

// jinf_rmsnorm_matvec_batch, jinf_rmsnorm_swiglu_matvec_batch and
// jinf_rmsnorm_qkv_rope_batch, first completing the pending residual add
// `pend` (may be null) into h: h[b] += sum of its partials, written back.
// The Q / K / V call also takes `part` (may be null; matvec_batch_defer_bytes
// for its rows, 16-byte aligned): when its columns are split, the splits'
// partial sums go there and a launch of its own sums them and applies the
// RoPE / cache-store epilogue, instead of the GEMV's last workgroup of each
// row group.  x_ready (Q/K/V): the previous Q/K/V call of this layer, on the
// same workspace and input, already prepared x (the preparation is skipped).
int rmsnorm_matvec_batch_m(const void* weight, int qtype, float* h, int ld_h, const void* norm_w,
                           int norm_type, float eps, float* y, int ld_y, int rows, int cols,
                           int n_batch, void* workspace, size_t workspace_bytes,
                           const MbDefer* pend, hipStream_t stream);
int rmsnorm_swiglu_matvec_batch_m(const void* w_gate, const void* w_up, int qtype, float* h,
                                  int ld_h, const void* norm_w, int norm_type, float eps, float* y,
                                  int ld_y, int n_ff, int cols, int n_batch, void* workspace,
                                  size_t workspace_bytes, const MbDefer* pend, hipStream_t stream);
int rmsnorm_qkv_rope_batch_m(const void* wq, const void* wk, const void* wv, int qtype, float* h,
                             int ld_h, const void* norm_w, int norm_type, float eps, int n_embd,
                             float* q, int ld_q, void* k_cache, void* v_cache, int kv_type,
                             int64_t ld_seq, const int32_t* positions, int max_ctx, int head_dim,
                             int n_heads, int n_heads_kv, float freq_base, int n_batch,
                             void* workspace, size_t workspace_bytes, const MbDefer* pend,
                             float* part, size_t part_bytes, bool x_ready, hipStream_t stream);

// A layer's Q / K / V projections whose matrices may be of up to three
// formats (w / types in q, k, v order): one GEMV launch per format, all
// reading the x the first one prepares (except Q6_K beyond 32 sequences,
// whose two one-tile launches prepare their own), their split partials laid
// one after another in `part` (qkv_defer_bytes), and one epilogue launch for
// all of them.  `pend` is merged ahead of the first launch.
int rmsnorm_qkv_rope_batch_mixed(const void* const w[3], const int types[3], float* h, int ld_h,
                                 const void* norm_w, int norm_type, float eps, int n_embd,
                                 float* q, int ld_q, void* k_cache, void* v_cache, int kv_type,
                                 int64_t ld_seq, const int32_t* positions, int max_ctx,
                                 int head_dim, int n_heads, int n_heads_kv, float freq_base,
                                 int n_batch, void* workspace, size_t workspace_bytes,
                                 const MbDefer* pend, float* part, size_t part_bytes,
                                 hipStream_t stream);

// Bytes of `part` that rmsnorm_qkv_rope_batch_mixed needs for these formats.
size_t qkv_defer_bytes(const int types[3], int q_dim, int kv_dim, int n_embd, int n_batch);

}  // namespace jinf
