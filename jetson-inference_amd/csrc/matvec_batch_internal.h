// Internal interface of the batched GEMVs for the batch decoder (not in the
// public headers): a residual add whose column-split partial sums are left
// for the next normed GEMV call to merge (a launch of its own ahead of that
// call's preparation), instead of being merged by the GEMV's last workgroup
// of each row group.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jinf {

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

// jinf_matvec_batch_add's products, with the residual add left pending in
// *out (part: matvec_batch_defer_bytes bytes, 16-byte aligned).  y is not
// touched: the next call below that takes `pend` with h = y first adds the
// partial sums into h (summed in split order, as the GEMV's own merge does),
// then normalizes.
int matvec_batch_add_defer(const void* weight, int qtype, const float* x, int ld_x, int rows,
                           int cols, int n_batch, float* part, size_t part_bytes, void* workspace,
                           size_t workspace_bytes, MbDefer* out, hipStream_t stream);

// jinf_rmsnorm_matvec_batch, jinf_rmsnorm_swiglu_matvec_batch and
// jinf_rmsnorm_qkv_rope_batch, first completing the pending residual add
// `pend` (may be null) into h: h[b] += sum of its partials, written back.
// The Q / K / V call also takes `part` (may be null; matvec_batch_defer_bytes
// for its rows, 16-byte aligned): when its columns are split, the splits'
// partial sums go there and a launch of its own sums them and applies the
// RoPE / cache-store epilogue, instead of the GEMV's last workgroup of each
// row group.
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
                             float* part, size_t part_bytes, hipStream_t stream);

}  // namespace jinf
