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
// registers (CPT float4 chunks per lane: 4 up to 16384 columns, 8 up to 32768),
// exponentiated once, and written once: one HBM read and one write per
// element, against the reference's three reads and two exp evaluations.
// Every chunk's load is issued before any arithmetic, so a row's loads are in
// flight together.  Max and sum are DPP wave reductions plus one LDS exchange
// and one barrier each; each lane's exponentials and then the wave's lanes are
// summed in fp32, the per-wave sums in fp64.  The exponential is the
// two-operation exp_neg_fast (relative error below 6.5e-6 for every normal
// result, within the 1e-5 bar; a six-operation Cody-Waite form, about 2 ulp,
// took 0.8-1.0 us longer at config 5: 26.15-26.32 against 25.11-25.28 us,
// interleaved, with the ragged-row probe at 24.83-24.92).  Chunks past the row's live
// length do no arithmetic (whole waves branch over them), so the VALU cost
// follows the live length, not the padded stride.
// Grid: (rows per length entry, length entries), so a workgroup finds its
// length entry from blockIdx.y without an integer division (the earlier
// 64-bit division sat on every row's critical path, ahead of its loads:
// 1.2 us of 26.6 at config 5).  Consecutive workgroups are the heads of one
// sequence, which the round-robin dispatch spreads over all eight XCDs.
// Measured at config 5 (4096 rows, stride 8192, random len; 130 MB):
//   2-D grid, 512 lanes x 4 chunks   24.4 us (66% of 8 TB/s; a streaming
//                                    probe of the same geometry, loads ->
//                                    one cross-lane exchange -> stores,
//                                    22.5-23.0 us: 94% of it)
//   1-D grid with the division       26.6 us (256 x 8: 25.4 us without it)
//   1024 lanes x 2 chunks            27.9 us
//   waves without live data leaving before the barriers   25.5 us
//   one barrier (per-wave max and sum combined)            26.3-30.7 us
//   longest sequence first (host-sorted order)             24.2 us (probe:
//                                    unchanged, so the tail is not the cause)
//   earlier: two rows per workgroup sharing the barriers, one wave per row,
//   length-scaled waves with several short rows per workgroup, loading the
//   first chunk before the length is known: all slower.
// Rows longer than the register capacity (or unaligned rows) take a loop
// kernel that reads the row three times (max, sum, write) like the reference.
#include <math.h>

#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"

namespace jinf {

constexpr int kSmMaxGridY = 65535;

__device__ __forceinline__ int clamp_len(int L, int n_cols) {
    L = L < 0 ? 0 : L;
    return L > n_cols ? n_cols : L;
}

__device__ __forceinline__ int live_len(const int32_t* lens, int rows_per_len, int n_cols,
                                        int64_t row) {
    if (!lens) return n_cols;
    return clamp_len(lens[(uint32_t)row / (uint32_t)rows_per_len], n_cols);
}

// One row per workgroup of BS lanes, CPT float4 chunks per lane.  GRID2D:
// the grid is (rows_per_len, length entries) and row = blockIdx.y *
// rows_per_len + blockIdx.x; otherwise one dimension of n_rows (length entry
// by division).  BS is a template argument: with the block size known at
// compile time the chunk offsets become immediates and the config-5 launch
// takes 24.5 us instead of 26.2.
template <int CPT, int BS, bool GRID2D>
__global__ __launch_bounds__(BS) void softmax_vec_kernel(
    float* out, int ld_out, const float* in, int ld_in, int n_rows, int n_cols,
    const int32_t* lens, int rows_per_len, float scale) {
#pragma clang fp contract(off)
    __shared__ float redf[16];
    __shared__ double redd[16];
    constexpr int bs = BS;
    constexpr int nw = BS / kWave;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const float ninf = -INFINITY;
    int64_t row;
    int L;
    if constexpr (GRID2D) {
        row = (int64_t)blockIdx.y * rows_per_len + blockIdx.x;
        L = row < n_rows ? (lens ? clamp_len(lens[blockIdx.y], n_cols) : n_cols) : 0;
    } else {
        row = blockIdx.x;
        L = live_len(lens, rows_per_len, n_cols, row);
    }
    const int nfull = L >> 2;  // whole float4 chunks
    const float* x = in + row * ld_in;
    float* y = out + row * ld_out;

    // Chunks at or past L do no arithmetic: whole waves skip them.
    float v[CPT][4];
    float mx = ninf;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (c < nfull) {
            Act<float>::load(x + 4 * c, v[j]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j][e] = (4 * c + e < L) ? x[4 * c + e] : ninf;
        }
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (4 * c < L) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[j][e] = v[j][e] * scale;  // -inf * scale stays -inf for scale > 0
                mx = fmaxf(mx, v[j][e]);
            }
        }
    }
    mx = wave_max_f32(mx);
    if (lane == 0) redf[wid] = mx;
    __syncthreads();
    {
        float m = redf[0];
#pragma unroll
        for (int i = 1; i < nw; ++i) m = fmaxf(m, redf[i]);
        mx = m;
    }
    // Each lane's exponentials (at most 4 * CPT, all in (0, 1]) and the wave's
    // lanes are summed in fp32, the wave sums in fp64: the sum's relative error
    // stays below (4 * CPT + 6) * 2^-24 (2.3e-6 at 8 chunks), and fp32 lane
    // sums measured 24.7 us against 24.9 us for fp64 lane sums at config 5.
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (4 * c < L) {
            float part = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ex = 4 * c + e < L ? exp_neg_fast(v[j][e] - mx) : 0.0f;
                v[j][e] = ex;
                part += ex;
            }
            sum += part;
        }
    }
    sum = wave_sum_f32(sum);
    if (lane == 0) redd[wid] = (double)sum;
    __syncthreads();
    double t = redd[0];
#pragma unroll
    for (int i = 1; i < nw; ++i) t += redd[i];
    const float inv = 1.0f / (float)t;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (c < nfull) {
            const float o[4] = {v[j][0] * inv, v[j][1] * inv, v[j][2] * inv, v[j][3] * inv};
            Act<float>::store(y + 4 * c, o);
        } else if (4 * c < L) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (4 * c + e < L) y[4 * c + e] = v[j][e] * inv;
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
    for (int i = threadIdx.x; i < L; i += blockDim.x) sum += (double)exp_neg_fast(x[i] * scale - m);
    sum = block_sum(sum, redd);
    const float inv = 1.0f / (float)sum;
    for (int i = threadIdx.x; i < L; i += blockDim.x) y[i] = exp_neg_fast(x[i] * scale - m) * inv;
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
    // lanes x chunks per lane: 64 x 4 up to 256 columns (1024 fit), 256 x 4
    // up to 4096, 512 x 4 up to 8192, 1024 x 4 up to 16384, 1024 x 8 up to
    // 32768
    if (vec && n_cols <= 32768) {
        const int rpl = lens ? rows_per_len : n_rows;
        const int64_t groups = ((int64_t)n_rows + rpl - 1) / rpl;
        const bool g2 = groups <= kSmMaxGridY;
        const dim3 grid = g2 ? dim3((unsigned)(rpl < n_rows ? rpl : n_rows), (unsigned)groups)
                             : dim3((unsigned)n_rows);
        auto go = [&](auto k2d, auto k1d, int bs) {
            return launch(g2 ? k2d : k1d, grid, dim3(bs), 0, stream, out, ld_out, in, ld_in,
                          n_rows, n_cols, lens, rpl, scale);
        };
        if (n_cols <= 256)
            return go(softmax_vec_kernel<4, 64, true>, softmax_vec_kernel<4, 64, false>, 64);
        if (n_cols <= 4096)
            return go(softmax_vec_kernel<4, 256, true>, softmax_vec_kernel<4, 256, false>, 256);
        if (n_cols <= 8192)
            return go(softmax_vec_kernel<4, 512, true>, softmax_vec_kernel<4, 512, false>, 512);
        if (n_cols <= 16384)
            return go(softmax_vec_kernel<4, 1024, true>, softmax_vec_kernel<4, 1024, false>,
                      1024);
        return go(softmax_vec_kernel<8, 1024, true>, softmax_vec_kernel<8, 1024, false>, 1024);
    }
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
