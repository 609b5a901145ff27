// Masked fp32 row softmax for gfx950.
//
// Semantics (reference cuda/softmax_kernel.cu:8-42; the live masked form is the
// softmax phase of cuda/attention_kernel.cu:59-87 over n_past = pos + 1
// scores):
//   s_j = scale * x_j                 for j < L (L = live length of the row)
//   m   = max_j s_j
//   e_j = exp(s_j - m)
//   y_j = e_j * (1 / sum_j e_j)
// Elements j >= L are neither read nor written.
//
// Design: one workgroup per row.  The live part of the row is loaded once into
// registers (kSmCPT float4 chunks per thread, so up to 32 KiB per row with
// 256 lanes), exponentiated once, and written once: one HBM read and one write
// per element, against the reference's three reads and two exp evaluations.
// Every chunk's load is issued before any arithmetic, so a row's loads are in
// flight together.  Max and sum are DPP wave reductions plus one LDS exchange
// and one barrier each; each aligned group of 4 exponentials is summed in fp32
// and the group sums in fp64.  Chunks past the row's live length do no
// arithmetic (whole waves branch over them), so the VALU cost follows the live
// length, not the padded stride.
// Measured at config 5 (4096 rows, stride 8192, random len): this form 26 us
// (63% of 8 TB/s); the earlier one with loads and maxima interleaved per chunk
// and two-barrier shuffle reductions 30 us.  Also slower: two rows per
// workgroup sharing the barriers (31 us), 2 or 16 chunks per lane instead of 8
// (4 equal), longest-first row order, one wave per row, length-scaled waves
// per row with several short rows per workgroup, loading the first chunk
// before the length is known.  At uniform 8192-long rows the earlier form
// reached 74% of 8 TB/s (a plain copy: 75%); ragged rows lose to the per-row
// latency chain.
// Rows longer than the register capacity (or unaligned rows) take a loop
// kernel that reads the row three times (max, sum, write) like the reference.
#include <math.h>

#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"

namespace jinf {

constexpr int kSmCPT = 8;  // float4 chunks per lane kept in registers

__device__ __forceinline__ int live_len(const int32_t* lens, int rows_per_len, int n_cols,
                                        int64_t row) {
    if (!lens) return n_cols;
    int L = lens[row / rows_per_len];
    L = L < 0 ? 0 : L;
    return L > n_cols ? n_cols : L;
}

// RPW rows per workgroup (rows RPW b .. RPW b + RPW - 1; the launches use 1):
// their loads are in flight together and their reductions share the
// workgroup's barriers.
template <int CPT = kSmCPT, int RPW = 1>
__global__ __launch_bounds__(1024) void softmax_vec_kernel(
    float* out, int ld_out, const float* in, int ld_in, int n_rows, int n_cols,
    const int32_t* lens, int rows_per_len, float scale) {
#pragma clang fp contract(off)
    __shared__ float redf[16 * RPW];
    __shared__ double redd[16 * RPW];
    const int bs = blockDim.x;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave, nw = bs / kWave;
    const float ninf = -INFINITY;
    int L[RPW], nfull[RPW];
    const float* x[RPW];
    float* y[RPW];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int64_t row = (int64_t)blockIdx.x * RPW + q;
        L[q] = row < n_rows ? live_len(lens, rows_per_len, n_cols, row) : 0;
        nfull[q] = L[q] >> 2;  // whole float4 chunks
        x[q] = in + row * ld_in;
        y[q] = out + row * ld_out;
    }

    // Chunks at or past L do no arithmetic: whole waves skip them.
    float v[RPW][CPT][4];
    float mx[RPW];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        mx[q] = ninf;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = threadIdx.x + j * bs;
            if (c < nfull[q]) {
                Act<float>::load(x[q] + 4 * c, v[q][j]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[q][j][e] = (4 * c + e < L[q]) ? x[q][4 * c + e] : ninf;
            }
        }
    }
#pragma unroll
    for (int q = 0; q < RPW; ++q)
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = threadIdx.x + j * bs;
            if (4 * c < L[q]) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[q][j][e] = v[q][j][e] * scale;  // -inf * scale stays -inf for scale > 0
                    mx[q] = fmaxf(mx[q], v[q][j][e]);
                }
            }
        }
    // one exchange for every row's maximum
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        mx[q] = wave_max_f32(mx[q]);
        if (lane == 0) redf[q * 16 + wid] = mx[q];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        float m = redf[q * 16];
        for (int i = 1; i < nw; ++i) m = fmaxf(m, redf[q * 16 + i]);
        mx[q] = m;
    }
    double sum[RPW];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        sum[q] = 0.0;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = threadIdx.x + j * bs;
            if (4 * c < L[q]) {
                float part = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float ex = 4 * c + e < L[q] ? exp_neg(v[q][j][e] - mx[q]) : 0.0f;
                    v[q][j][e] = ex;
                    part += ex;
                }
                sum[q] += (double)part;
            }
        }
    }
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        sum[q] = wave_sum_f64(sum[q]);
        if (lane == 0) redd[q * 16 + wid] = sum[q];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        double t = redd[q * 16];
        for (int i = 1; i < nw; ++i) t += redd[q * 16 + i];
        const float inv = 1.0f / (float)t;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = threadIdx.x + j * bs;
            if (c < nfull[q]) {
                const float o[4] = {v[q][j][0] * inv, v[q][j][1] * inv, v[q][j][2] * inv,
                                    v[q][j][3] * inv};
                Act<float>::store(y[q] + 4 * c, o);
            } else if (4 * c < L[q]) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * c + e < L[q]) y[q][4 * c + e] = v[q][j][e] * inv;
            }
        }
    }
}

// Any length / alignment: pass 1 max, pass 2 sum of exponentials, pass 3
// write; each pass re-reads the row.
__global__ __launch_bounds__(1024) void softmax_loop_kernel(
    float* out, int ld_out, const float* in, int ld_in, int n_cols, const int32_t* lens,
    int rows_per_len, float scale) {
#pragma clang fp contract(off)
    __shared__ float redf[16];
    __shared__ double redd[16];
    const int64_t row = blockIdx.x;
    const int L = live_len(lens, rows_per_len, n_cols, row);
    if (L == 0) return;
    const float* x = in + row * ld_in;
    float* y = out + row * ld_out;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < L; i += blockDim.x) m = fmaxf(m, x[i] * scale);
    m = block_max(m, redf);
    double sum = 0.0;
    for (int i = threadIdx.x; i < L; i += blockDim.x) sum += (double)exp_neg(x[i] * scale - m);
    sum = block_sum(sum, redd);
    const float inv = 1.0f / (float)sum;
    for (int i = threadIdx.x; i < L; i += blockDim.x) y[i] = exp_neg(x[i] * scale - m) * inv;
}

static int softmax_dispatch(float* out, int ld_out, const float* in, int ld_in, int n_rows,
                            int n_cols, const int32_t* lens, int rows_per_len, float scale,
                            hipStream_t stream) {
    if (n_rows < 0 || n_cols < 0) return JINF_HIP_ERR_INVALID;
    if (n_rows == 0 || n_cols == 0) return JINF_HIP_OK;
    if (!out || !in || ld_out < n_cols || ld_in < n_cols) return JINF_HIP_ERR_INVALID;
    if (lens && rows_per_len <= 0) return JINF_HIP_ERR_INVALID;
    if (!(scale > 0.0f) || !isfinite(scale)) return JINF_HIP_ERR_INVALID;
    const bool vec = aligned(out, 16) && aligned(in, 16) && ld_out % 4 == 0 && ld_in % 4 == 0;
    const int nch = (n_cols + 3) / 4;
    int bs = round_up((nch + kSmCPT - 1) / kSmCPT, kWave);
    if (bs < 256 && n_cols > 256) bs = 256;
    if (bs < kWave) bs = kWave;
    if (vec && bs <= 1024)
        return launch(softmax_vec_kernel<kSmCPT, 1>, dim3(n_rows), dim3(bs), 0, stream, out,
                      ld_out, in, ld_in, n_rows, n_cols, lens, rows_per_len, scale);
    const int lbs = n_cols >= 1024 ? 1024 : round_up(n_cols, kWave);
    return launch(softmax_loop_kernel, dim3(n_rows), dim3(lbs), 0, stream, out, ld_out, in,
                  ld_in, n_cols, lens, rows_per_len, scale);
}

}  // namespace jinf

extern "C" int jinf_softmax_rows_f32(float* out, int ld_out, const float* in, int ld_in,
                                     int n_rows, int n_cols, const int32_t* lens,
                                     int rows_per_len, float scale, hipStream_t stream) {
    return jinf::softmax_dispatch(out, ld_out, in, ld_in, n_rows, n_cols, lens, rows_per_len,
                                  scale, stream);
}

// Drop-in for cuda/softmax_kernel.cu:46-51 (one fp32 row; output may alias input).
extern "C" void jinf_cuda_softmax(float* output, const float* input, int n, hipStream_t stream) {
    if (n <= 0) return;
    if (jinf::softmax_dispatch(output, n, input, n, 1, n, nullptr, 1, 1.0f, stream) ==
        JINF_HIP_ERR_INVALID)
        JINF_LOG("jinf_cuda_softmax: invalid argument (n=%d)", n);
}
