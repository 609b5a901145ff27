// Batched dequant-GEMV on the matrix cores: the reference's per-token
// matrix-vector products (cuda/matmul_kernels.cu:8-225, called per token at
// src/engine.cpp:429-508) for up to 64 sequences decoded together, so that
// every weight byte read from HBM serves all of them.
//
//   y[b, r] = sum_c W[r, c] x[b, c]        b < n_batch, W in Q4_0 / Q8_0 /
//                                          Q4_K / Q6_K blocks along c
//
// Arithmetic.  The products run on v_mfma_f32_32x32x16_f16 (A = 32 tokens x
// 16 columns, B = 16 columns x 32 weight rows, fp32 accumulate):
//   - B holds the weights' integer codes, exact in fp16: q - 8 (Q4_0), q
//     (Q8_0), sc * q <= 945 (Q4_K, the 6-bit sub-block scale folded in) and
//     q - 32 (Q6_K); the block scales multiply the fp32 partial sums;
//   - A holds x * s split into fp16 hi + lo (hi = fp16(v), lo = fp16(v - hi)),
//     s a power of two per token that puts the row's largest |x| in
//     [2^14, 2^15): about 22 significant bits for every element down to
//     2^-18 of that largest one, fp16's range never exceeded, and the 1/s
//     applied exactly to each slab's fp32 sum;
//   - Q4_K's minimum term dmin * m * sum(x) uses per-(token, sub-block) sums
//     of the scaled x.
// The result equals the fp32 dot product up to the fp32 rounding of the sums
// (the order differs from the reference's sequential sum).
//
// Data movement.  A preparation launch turns x (RMSNorm applied first when
// the GEMV reads a normed input, exactly as jinf_rmsnorm_rows computes it)
// into per-slab records of MFMA fragments (below).  A GEMV workgroup (4
// waves for up to 32 sequences, 8 for two M-tiles) owns 64 weight rows (two
// 32-row tiles) and a range of 256-column slabs.  Per slab its lanes copy,
// with direct-to-LDS loads, the 64 rows' bytes (the aligned 16-byte chunks
// covering each row's slab: with a 16-byte aligned matrix they start inside
// it and end before the next 16-byte boundary past its last byte) into the
// workgroup's LDS slot, one slab ahead of the matrix-core work, and each
// wave loads its own k-steps' x fragments into registers (Q6_K: the x
// record goes into the slot too).  Wave w multiplies k-steps 4 w .. 4 w + 3
// (2 w .. 2 w + 1 with 8 waves) of the slab for both row tiles, and the
// waves' sums are added in LDS at the end.
// Within a 16-column k-step, lane l supplies token / row l % 32 and columns
// 8 (l / 32) .. + 7 in the order (0, 4, 1, 5, 2, 6, 3, 7), the order in
// which four bytes of packed 4-bit codes unpack into fp16 pairs with two
// masks; A uses the same order, so each fragment is one 16-byte LDS read.
//
// Split over the columns.  Small row counts give few workgroups, so the
// slabs are split over k_splits workgroups per row group; each writes its
// fp32 partial to the workspace with device-coherent stores and bumps the
// group's counter, and the last one sums the partials in split order (the
// result does not depend on which finished last), applies the epilogue and
// resets the counter to zero.
//
// Epilogues (per output row r, token b): store; add into y (the residual
// stream); SiLU(gate) * up for a gate / up pair; RoPE at the token's position
// and the K / V cache stores for fused q / k / v rows.
#include <hip/hip_runtime.h>
#include <math.h>

#include <type_traits>

#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels_ext.h"
#include "matvec_batch_internal.h"
#include "quant_device.h"
#include "rope_device.h"

namespace jinf {
namespace {

typedef _Float16 mb_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mb_h2 __attribute__((ext_vector_type(2)));
typedef float mb_f16 __attribute__((ext_vector_type(16)));
typedef float mb_f4 __attribute__((ext_vector_type(4)));

// Cache policy of the split partials' buffer accesses: sc1, device-coherent
// across the XCDs' L2s (as agent-scope atomics are).
constexpr int kMbSc1 = 16;

constexpr int kMbCols = 256;      // columns per slab
constexpr int kMbMaxBatch = 64;

enum MbEpi { kMbEpiStore = 0, kMbEpiAdd = 1, kMbEpiSwiGLU = 2, kMbEpiQKV = 3 };

// Bytes of one row's 256-column slab.
template <int QT> struct MbFmt;
template <> struct MbFmt<kQ4_0> { static constexpr int SB = 144; };
template <> struct MbFmt<kQ8_0> { static constexpr int SB = 272; };
template <> struct MbFmt<kQ4_K> { static constexpr int SB = 144; };
template <> struct MbFmt<kQ6_K> { static constexpr int SB = 210; };
// 16-byte chunks that cover one row's slab: Q4_0, Q8_0 and Q4_K slabs
// (144 / 272 / 144 bytes) start 16-byte aligned in a 16-byte aligned matrix;
// a Q6_K slab (210 bytes) starts at an even offset, so 14 chunks cover it.
template <int QT> constexpr int mb_nch() { return QT == kQ6_K ? 14 : MbFmt<QT>::SB / 16; }

// The fields the GEMV's first weight and x loads need come first: the first
// 14 dwords of the kernel arguments arrive preloaded in SGPRs.
struct MbJob {
    int rows;              // virtual rows; kMbEpiSwiGLU: output rows
    int n_slabs, n_groups, slabs_per_split;
    const uint8_t* W[3];   // segment matrices (same format and width)
    int64_t row_bytes;
    const uint8_t* xrec;   // prepared x records [n_slabs][mb_rec(MT)]
    int seg_end[3];        // virtual row where each segment ends
    int k_splits;
    const float* x;        // [n_batch][ld_x]
    int ld_x, n_batch;
    float* y;              // [n_batch][ld_y]
    int ld_y;
    void* kc;              // kMbEpiQKV: caches [n_batch][ld_seq], rows [max_ctx][kv_dim]
    void* vc;
    const int32_t* pos;    // kMbEpiQKV: [n_batch] positions (outside [0, max_ctx): no store)
    int kv_f16, kv_dim, head_dim, max_ctx;
    int64_t ld_seq;
    float* part;           // split partials [n_groups][k_splits][2 * MT * 1024]
    uint32_t* counters;    // [n_groups]
    float* dpart;          // kMbEpiAdd, deferred: partial sums [k_splits][n_batch][rows]
    int64_t dstride;       // (split stride), merged by the next preparation
    int x_ready;           // (host) x already prepared in xrec: no preparation launch
};

struct MbNoTheta {};
template <int EPI>
using MbTheta = typename std::conditional<EPI == kMbEpiQKV, RopeTheta, MbNoTheta>::type;

// Weight row `local` of workgroup `group` (ROWS rows per workgroup), clamped
// to the last row.  kMbEpiSwiGLU: the first ROWS / 2 are gate rows, the next
// ROWS / 2 the same rows of the up matrix.
template <int EPI, int ROWS>
__device__ __forceinline__ const uint8_t* mb_row(const MbJob& j, int group, int local) {
    if constexpr (EPI == kMbEpiSwiGLU) {
        constexpr int HALF = ROWS / 2;
        int r = group * HALF + local % HALF;
        if (r >= j.rows) r = j.rows - 1;
        return (local < HALF ? j.W[0] : j.W[1]) + (int64_t)r * j.row_bytes;
    } else {
        int v = group * ROWS + local;
        if (v >= j.rows) v = j.rows - 1;
        // selects, not an index into the job's arrays (which would place the
        // kernel argument in scratch memory)
        const uint8_t* base = v < j.seg_end[0] ? j.W[0] : v < j.seg_end[1] ? j.W[1] : j.W[2];
        const int start = v < j.seg_end[0] ? 0 : v < j.seg_end[1] ? j.seg_end[0] : j.seg_end[1];
        return base + (int64_t)(v - start) * j.row_bytes;
    }
}

// Two 16-bit LDS reads (2-byte aligned) as one word.  (One 32-bit read at
// the 2-byte aligned address gives the same word, but unaligned LDS reads
// are slower: 116 against 111 us over the four batch-32 GEMVs of a layer.)
__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

__device__ __forceinline__ mb_h2 as_h2(uint32_t u) { return __builtin_bit_cast(mb_h2, u); }

// Eight 4-bit codes (four bytes, element 2 i in the low nibble of byte i)
// as fp16 (q + bias) in the order (0, 4, 1, 5, 2, 6, 3, 7); `hi2` adds two
// high bits per element (Q6_K: the pair masks of element i and i + 4).
__device__ __forceinline__ mb_h8 mb_nibbles(uint32_t w, uint32_t hi2, float bias) {
    const mb_h2 b = mb_h2{(_Float16)(-1024.0f + bias), (_Float16)(-1024.0f + bias)};
    mb_h2 p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // (w >> 4 i) & 0x000F000F | 0x64006400 in one instruction
        uint32_t v = __builtin_amdgcn_bitop3_b32(w >> (4 * i), 0x000F000Fu, 0x64006400u, 0xEA);
        v |= ((hi2 >> (2 * i)) & 0x00030003u) << 4;
        p[i] = as_h2(v) + b;  // (1024 + q) + (bias - 1024): exact
    }
    return mb_h8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// Eight 4-bit codes q times an integer sub-block scale g <= 63 as fp16 g q,
// in the order of mb_nibbles: one packed FMA per pair, (1024 + q) g +
// (-1024 g), whose exact value g q <= 945 is representable, so its one
// rounding changes nothing.
__device__ __forceinline__ mb_h8 mb_nibbles_scaled(uint32_t w, _Float16 g) {
    const mb_h2 g2 = mb_h2{g, g};
    const mb_h2 c = mb_h2{(_Float16)-1024.0f, (_Float16)-1024.0f} * g2;  // exact: g < 64
    mb_h2 p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = __builtin_amdgcn_bitop3_b32(w >> (4 * i), 0x000F000Fu, 0x64006400u, 0xEA);
        p[i] = __builtin_elementwise_fma(as_h2(v), g2, c);
    }
    return mb_h8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// Eight int8 codes (two words) as fp16 in the order (0, 4, 1, 5, 2, 6, 3, 7).
__device__ __forceinline__ mb_h8 mb_int8(uint32_t w0, uint32_t w1) {
    const mb_h2 b = mb_h2{(_Float16)-1152.0f, (_Float16)-1152.0f};
    mb_h2 p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // byte i of w0 -> byte 0, byte i of w1 -> byte 2, zero elsewhere
        const uint32_t sel = (uint32_t)i | 0x0C00u | ((uint32_t)(4 + i) << 16) | 0x0C000000u;
        const uint32_t v = __builtin_amdgcn_perm(w1, w0, sel);
        p[i] = as_h2((v ^ 0x00800080u) | 0x64006400u) + b;  // 1024 + (q + 128) - 1152
    }
    return mb_h8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

__device__ __forceinline__ mb_f16 mfma(mb_h8 a, mb_h8 b, mb_f16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Token of accumulator register r in lane half h of M-tile mt
// (v_mfma_f32_32x32x* D layout: row 8 (r / 4) + 4 h + r % 4).
__device__ __forceinline__ int mb_token(int mt, int r, int h) {
    return 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
}

// ---- x preparation ----
//
// One record per 256-column slab, in the order the GEMVs read it:
//   [MT M-tiles][16 k-steps][hi, lo][64 lanes] 16-byte fragments, lane
//   (token % 32) + 32 h holding columns 16 t + 8 h .. + 7 in the order
//   (0, 4, 1, 5, 2, 6, 3, 7);
//   then the slab data: inv_s[32 MT] (1/s per token, the same in every slab)
//   and Q4_K's xs[8 sub-blocks][32 MT tokens] (sums of the scaled x over 32
//   columns).
__host__ __device__ constexpr int mb_meta(int mt) { return 2048 * mt; }
__host__ __device__ constexpr int mb_rec(int mt) { return mt * 32768 + mb_meta(mt); }
static_assert(mb_rec(1) == mb_rec_bytes(1) && mb_rec(2) == mb_rec_bytes(2), "record layout");

constexpr int kMbMaxCols = 32768;                 // columns the preparation holds

// grid (ceil(n_slabs / 8), 32 MT): workgroup (c, b) converts slabs 8 c ..
// 8 c + 7 of token b.  Each holds token b's whole row in registers (thread i
// takes the 8-column groups i, i + 256, ...; every workgroup of the token
// reads the row, mostly from L2) for the row's one reduction; tokens >=
// n_batch get zeros and unit scale.  With norm_w the row is first
// RMS-normalised exactly as jinf_rmsnorm_rows does (x^ = fl32(fl32(x rs) g)).
// One power of two s per token puts max |x^ s| in [2^14, 2^15): hi =
// fp16(x^ s) and lo = fp16(x^ s - hi) then carry about 22 significant bits
// of every element (lo reaches fp16's subnormals only below 2^-18 of the
// row's largest element), and fp16's range is never exceeded.
// RMSNorm weights of 8-column group g (1 without a norm): 16-byte loads when
// the weights are 16-byte aligned, else element loads.
__device__ __forceinline__ void mb_norm8(const void* norm_w, int norm_f16, int g, float (&gw)[8]) {
    if (!norm_w) {
#pragma unroll
        for (int e = 0; e < 8; ++e) gw[e] = 1.0f;
    } else if (((uintptr_t)norm_w & 15) != 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            gw[e] = norm_f16 ? h2f(static_cast<const uint16_t*>(norm_w)[8 * g + e])
                             : static_cast<const float*>(norm_w)[8 * g + e];
    } else if (norm_f16) {
        const uint4 q = *(static_cast<const uint4*>(norm_w) + g);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            gw[2 * i] = h2f((uint16_t)(w[i] & 0xFFFFu));
            gw[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
        }
    } else {
        const float4 p = *(static_cast<const float4*>(norm_w) + 2 * g);
        const float4 q = *(static_cast<const float4*>(norm_w) + 2 * g + 1);
        gw[0] = p.x; gw[1] = p.y; gw[2] = p.z; gw[3] = p.w;
        gw[4] = q.x; gw[5] = q.y; gw[6] = q.z; gw[7] = q.w;
    }
}

// KG: 8-column groups per thread (the row's groups over 256 threads: 2 at
// 4096 columns, 7 of 8 at 14336).  Every x and norm-weight load is issued
// before any arithmetic (weights held in registers for KG <= 8), and the two
// row reductions are DPP wave reductions with one LDS exchange.
// chunk_slabs > 0: workgroup (c, b) reads and converts only slabs c
// chunk_slabs .. + chunk_slabs - 1.  Without row statistics (no norm only)
// that chunk is its whole row, so the scale s is per chunk: the GEMV splits
// its columns in the same chunks and takes each split's 1 / s from its first
// slab's record.  With row statistics st_ss / st_mx ([n_batch][st_n]: the
// sums of squares and largest |x g| of the row's slices, written by the
// residual merge that produced x) the whole row's reduction is read from
// them instead, in slice order.
template <int MT, int KG>
__global__ __launch_bounds__(256) void mb_prepare_kernel(const float* __restrict__ x, int ld_x,
                                                          int n_batch, int cols,
                                                          const void* __restrict__ norm_w,
                                                          int norm_f16, float eps,
                                                          uint8_t* __restrict__ rec,
                                                          int chunk_slabs,
                                                          const double* __restrict__ st_ss,
                                                          const float* __restrict__ st_mx,
                                                          int st_n) {
    __shared__ double red[4];
    __shared__ float redf[4];
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int row_cols = cols;
    int c0 = 0;                // first column of this workgroup's row
    int sel = blockIdx.x;      // which of each thread's groups it converts (-1: all)
    if (chunk_slabs > 0) {
        c0 = blockIdx.x * chunk_slabs * kMbCols;
        cols = min(cols - c0, chunk_slabs * kMbCols);
        rec += (int64_t)blockIdx.x * chunk_slabs * mb_rec(MT);
        sel = -1;
    }
    const int ng = cols / 8;  // a multiple of 32
    const bool live = b < n_batch;
    const float* xr = x + (int64_t)(live ? b : 0) * ld_x + c0;
    const int g0 = c0 / 8;  // norm-weight group of this row's first column
    constexpr bool GW_EARLY = KG <= 8;
    float v[KG][8];
    float gwr[GW_EARLY ? KG : 1][8];
#pragma unroll
    for (int k = 0; k < KG; ++k) {
        const int g = tid + 256 * k;
        if (live && g < ng) {
            const float4 p = *reinterpret_cast<const float4*>(xr + 8 * g);
            const float4 q = *reinterpret_cast<const float4*>(xr + 8 * g + 4);
            v[k][0] = p.x; v[k][1] = p.y; v[k][2] = p.z; v[k][3] = p.w;
            v[k][4] = q.x; v[k][5] = q.y; v[k][6] = q.z; v[k][7] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[k][e] = 0.0f;
        }
    }
    if constexpr (GW_EARLY) {
#pragma unroll
        for (int k = 0; k < KG; ++k) {
            const int g = tid + 256 * k;
            if (g < ng) {
                mb_norm8(norm_w, norm_f16, g0 + g, gwr[k]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) gwr[k][e] = 1.0f;
            }
        }
    }
    auto gweights = [&](int k, int g, float (&gw)[8]) {
        if constexpr (GW_EARLY) {
#pragma unroll
            for (int e = 0; e < 8; ++e) gw[e] = gwr[k][e];
        } else {
            mb_norm8(norm_w, norm_f16, g0 + g, gw);
        }
    };
    // one workgroup reduction: the sum of squares (norm_w) and the largest
    // |x g| (|x| without norm_w); max |x^| <= rs max |x g| up to a few
    // roundings, so rs max |x g| fixes the scale (|x^ s| stays below
    // 2^15 (1 + 2^-21), far inside fp16's range)
    double ss = 0.0;
    float m = 0.0f;
    if (st_ss) {
        // the row's reduction, done by the merge that wrote x
        if (live) {
            for (int i = 0; i < st_n; ++i) {
                ss += st_ss[(int64_t)b * st_n + i];
                m = fmaxf(m, st_mx[(int64_t)b * st_n + i]);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < KG; ++k) {
            const int g = tid + 256 * k;
            if (g < ng) {
                float gw[8];
                gweights(k, g, gw);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (norm_w) ss = fma((double)v[k][e], (double)v[k][e], ss);
                    m = fmaxf(m, fabsf(v[k][e] * gw[e]));
                }
            }
        }
        ss = wave_sum_f64(ss);
        m = wave_max_f32(m);
        if ((tid & (kWave - 1)) == 0) {
            red[tid / kWave] = ss;
            redf[tid / kWave] = m;
        }
        __syncthreads();
        ss = red[0];
        m = redf[0];
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            ss += red[i];
            m = fmaxf(m, redf[i]);
        }
    }
    if (norm_w && live) {
        const float rs = rms_scale(ss, row_cols, eps);
        m = rs * m;
#pragma unroll
        for (int k = 0; k < KG; ++k) {
            const int g = tid + 256 * k;
            if (g < ng && (sel < 0 || k == sel)) {  // only this workgroup's groups
#pragma clang fp contract(off)
                float gw[8];
                gweights(k, g, gw);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[k][e] = (v[k][e] * rs) * gw[e];
            }
        }
    }
    const int ex = mb_scale_exp(m);
    const float sc = ldexpf(1.0f, 15 - ex);
#pragma unroll
    for (int k = 0; k < KG; ++k) {
        const int g = tid + 256 * k;
        // this workgroup's 256 groups (uniform over aligned groups of 32 threads)
        const bool here = g < ng && (sel < 0 || k == sel);
        const int slab = g >> 5, gi = g & 31;
        uint8_t* r = rec + (int64_t)slab * mb_rec(MT);
        float sum = 0.0f;
        if (here) sum = mb_put_group(r, b, gi, v[k], sc);
        // Q4_K sub-block sums: threads 4 q .. 4 q + 3 hold sub-block q's 32 columns
        sum += __shfl_xor(sum, 1, kWave);
        sum += __shfl_xor(sum, 2, kWave);
        if (here) mb_put_meta(r, MT, b, gi, sum, ex);
    }
}

// ---- merge of a deferred residual add ----
//
// h[b][c] += p_0[b][c] + p_1[b][c] + ... (split order, the order of the
// GEMV's own merge) for the k partial arrays p_s = part + s * stride of a
// deferred residual add ([n_batch][cols], cols a multiple of 256).  Grid
// (slices of 2048 columns, n_batch), one lane per 8 columns, every
// partial's load issued before the sums.  It also reduces each slice of the
// new row for the preparation that follows: the fp64 sum of squares and the
// largest |h g| (g the RMSNorm weights, or 1), the preparation's own
// per-element terms, into ss_out / mx_out [n_batch][slices].  (Folding the
// merge into the preparation, one workgroup per sequence so that the
// in-place update had no reader elsewhere, took 10.5 us per launch: one
// CU's outstanding loads bound the partials' read.)
constexpr int kMbSliceCols = 2048;
__global__ __launch_bounds__(256) void mb_merge_kernel(float* __restrict__ h, int ld_h,
                                                       int n_batch, int cols,
                                                       const float* __restrict__ part, int k,
                                                       int64_t stride,
                                                       const void* __restrict__ norm_w,
                                                       int norm_f16, double* __restrict__ ss_out,
                                                       float* __restrict__ mx_out) {
    __shared__ double red[4];
    __shared__ float redf[4];
    constexpr int SB = 8;  // partials loaded together
    const int b = blockIdx.y, tid = threadIdx.x;
    const int g = blockIdx.x * (kMbSliceCols / 8) + tid;  // 8-column group
    double ss = 0.0;
    float m = 0.0f;
    if (g < cols / 8) {
        float* hp = h + (int64_t)b * ld_h + 8 * g;
        const float* pp = part + (int64_t)b * cols + 8 * g;
        float v[8];
        {
            const float4 p = *reinterpret_cast<const float4*>(hp);
            const float4 q = *reinterpret_cast<const float4*>(hp + 4);
            v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
            v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
        }
        float gw[8];
        mb_norm8(norm_w, norm_f16, g, gw);
        float sum[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < k; s0 += SB) {
            float4 pv[SB][2];
#pragma unroll
            for (int u = 0; u < SB; ++u)
                if (s0 + u < k) {
                    pv[u][0] = *reinterpret_cast<const float4*>(pp + (s0 + u) * stride);
                    pv[u][1] = *reinterpret_cast<const float4*>(pp + (s0 + u) * stride + 4);
                }
#pragma unroll
            for (int u = 0; u < SB; ++u)
                if (s0 + u < k) {
                    sum[0] += pv[u][0].x; sum[1] += pv[u][0].y;
                    sum[2] += pv[u][0].z; sum[3] += pv[u][0].w;
                    sum[4] += pv[u][1].x; sum[5] += pv[u][1].y;
                    sum[6] += pv[u][1].z; sum[7] += pv[u][1].w;
                }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[e] = v[e] + sum[e];
            if (norm_w) ss = fma((double)v[e], (double)v[e], ss);
            m = fmaxf(m, fabsf(v[e] * gw[e]));
        }
        *reinterpret_cast<float4*>(hp) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(hp + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    ss = wave_sum_f64(ss);
    m = wave_max_f32(m);
    if ((tid & (kWave - 1)) == 0) {
        red[tid / kWave] = ss;
        redf[tid / kWave] = m;
    }
    __syncthreads();
    if (tid == 0) {
        ss = red[0];
        m = redf[0];
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            ss += red[i];
            m = fmaxf(m, redf[i]);
        }
        ss_out[(int64_t)b * gridDim.x + blockIdx.x] = ss;
        mx_out[(int64_t)b * gridDim.x + blockIdx.x] = m;
    }
}

// ---- the Q / K / V epilogue ----
//
// Virtual rows v0, v0 + 1 (a RoPE pair) of sequence b: q rows are rotated at
// the sequence's position and stored into y; k rows are rotated and v rows
// kept, each stored into the sequence's cache row at that position (a
// position outside [0, max_ctx) stores nothing).
__device__ __forceinline__ void mb_qkv_store(const MbJob& j, const RopeTheta& th, int b, int v0,
                                             float a, float c) {
    const int sgi = v0 < j.seg_end[0] ? 0 : v0 < j.seg_end[1] ? 1 : 2;
    const int local = v0 - (sgi == 0 ? 0 : j.seg_end[sgi - 1]);
    const int pos = j.pos[b];
    if (sgi < 2) {
        const float2 cs = rope_cs(pos, th.t[(local % j.head_dim) / 2]);
        rot(a, c, cs.x, cs.y);
    }
    if (sgi == 0) {
        float* yp = j.y + (int64_t)b * j.ld_y + local;
        yp[0] = a;
        yp[1] = c;
    } else if (pos >= 0 && pos < j.max_ctx) {
        const int64_t ci = (int64_t)b * j.ld_seq + (int64_t)pos * j.kv_dim + local;
        void* cp = sgi == 1 ? j.kc : j.vc;
        if (j.kv_f16) {
            uint16_t* p = static_cast<uint16_t*>(cp) + ci;
            p[0] = f2h(a);
            p[1] = f2h(c);
        } else {
            float* p = static_cast<float*>(cp) + ci;
            p[0] = a;
            p[1] = c;
        }
    }
}

// The deferred Q / K / V launches of one layer, one per weight format (q, k
// and v may each have their own), finished by one epilogue launch: (sequence,
// row pair) items [pairs[g - 1], pairs[g]) belong to job g.
struct MbQkvJobs {
    int pairs[3];  // first: each lane's first test needs them
    int n;
    MbJob j[3];
};

// The Q / K / V epilogue after deferred column splits: one lane per row pair
// of one sequence of one job sums that job's k_splits partials in split order
// (the order of the GEMV's own merge), then rotates and stores as above.
__global__ __launch_bounds__(256) void mb_qkv_epilogue_kernel(MbQkvJobs js, RopeTheta th) {
    constexpr int SB = 8;  // partials loaded together
    int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= js.pairs[js.n - 1]) return;
    // the job of item i (a wave-uniform choice except at job boundaries)
    const int g = i < js.pairs[0] ? 0 : (i < js.pairs[1] || js.n < 3) ? 1 : 2;
    if (g > 0) i -= js.pairs[g - 1];
    const MbJob& j = js.j[g];
    const int half = j.rows / 2;
    const int b = i / half, v0 = 2 * (i % half);
    const float* pp = j.dpart + (int64_t)b * j.rows + v0;
    float a = 0.0f, c = 0.0f;
    for (int s0 = 0; s0 < j.k_splits; s0 += SB) {
        float2 p[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u)
            if (s0 + u < j.k_splits) p[u] = *reinterpret_cast<const float2*>(pp + (s0 + u) * j.dstride);
#pragma unroll
        for (int u = 0; u < SB; ++u)
            if (s0 + u < j.k_splits) {
                a += p[u].x;
                c += p[u].y;
            }
    }
    mb_qkv_store(j, th, b, v0, a, c);
}

// ---- the GEMV ----
//
// Per 256-column slab a workgroup copies, with direct-to-LDS loads, its
// weight rows' bytes (the aligned 16-byte chunks covering each row's slab)
// and the slab's prepared x record into one of NBUF LDS slots; with NBUF > 1
// loads run NBUF - 1 slabs ahead of the matrix-core work (the launches use
// one slot, so a slab's loads are issued after the previous slab's product).
// Workgroup shapes: NT 32-row tiles (ROWS = 32 NT weight rows) and WV waves;
// the 16 k-steps of a slab are split into KSW parts, wave w taking k-part
// w / (WV / KSW) of TPW = NT KSW / WV tiles.  The launches use 64 rows (NT
// 2): one M-tile with WV 4, KSW 4 (each wave both tiles over 4 k-steps), two
// M-tiles with WV 8, KSW 8 (each wave both tiles over 2 k-steps, so that two
// M-tiles of x fragments fit in its registers beside their accumulators:
// 214 VGPRs, batch-64 step 6.62 -> 6.26 ms against WV 4 with x through LDS;
// at one M-tile the 8-wave shape measured the same as the 4-wave one).
// (8-wave shapes over 128 or 256 rows sharing each x record, with two slots
// so that the next slab's weights are in flight during the matrix-core work,
// measured slower.)
// Where the x fragments go: straight into registers, each wave its own
// k-steps' fragments; for Q6_K (whose decode needs more registers) through
// the LDS slot with the weights.
template <int QT, int MT> constexpr bool mb_xlds() { return QT == kQ6_K; }
// LDS slot: the weight chunks (NWI KiB), then the record's x fragments and
// sums (x through LDS) or, for Q4_K, only its x sums (NXI KiB), filled by
// 1 KiB direct-to-LDS instructions dealt round-robin to the waves.
template <int QT, int NT> constexpr int mb_nwi() { return (32 * NT * mb_nch<QT>() * 16 + 1023) / 1024; }
template <int QT, int MT> constexpr int mb_nxi() {
    return mb_xlds<QT, MT>() ? mb_rec(MT) / 1024 : QT == kQ4_K ? mb_meta(MT) / 1024 : 0;
}
template <int QT, int MT, int NT> constexpr int mb_slot() {
    return (mb_nwi<QT, NT>() + mb_nxi<QT, MT>()) * 1024;
}
// weight slots (slabs whose weights are in LDS or in flight; one slot when
// x goes through LDS) and x register sets (slabs whose fragments are in
// registers or in flight)
template <int QT, int MT> constexpr int mb_nbuf() { return mb_xlds<QT, MT>() ? 1 : 2; }
template <int QT, int MT> constexpr int mb_xbuf() { return mb_xlds<QT, MT>() ? 1 : 2; }
constexpr int mb_lcm(int a, int b) { return a % b == 0 ? a : b % a == 0 ? b : a * b; }
// LDS of a launch: the slots, reused after the loop for the KSW k-parts'
// sums (KSW NT MT 1024 floats)
template <int QT, int MT, int NT, int KSW> constexpr int mb_lds_bytes() {
    return mb_nbuf<QT, MT>() * mb_slot<QT, MT, NT>() > (KSW * NT * MT * 4096) ? mb_nbuf<QT, MT>() * mb_slot<QT, MT, NT>()
                                                                         : (KSW * NT * MT * 4096);
}
// loads per lane per slab for wave w of WV
constexpr int mb_share(int n, int w, int wv) { return (n - w + wv - 1) / wv; }

// Wait until this wave's LDS loads of the current step have landed: the
// NBUF - 2 later steps' loads (NXL x register loads and the wave's share of
// the slot's instructions per step) may still be in flight (none with one
// slot: its loads are issued in the step itself).
template <int NWI, int NXI, int NXL, int NBUF, int WV, int W = 0>
__device__ __forceinline__ void mb_wait_w(int wave) {
    if constexpr (NBUF == 1) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
    } else if constexpr (W < WV) {
        if (wave == W) {
            constexpr int n = (NBUF - 2) * (NXL + mb_share(NWI, W, WV) + mb_share(NXI, W, WV));
            __builtin_amdgcn_s_waitcnt(waitcnt_vm<n>());
            return;
        }
        mb_wait_w<NWI, NXI, NXL, NBUF, WV, W + 1>(wave);
    }
}

template <int MT> constexpr int mb_occ() { return 2; }  // waves per SIMD the kernel is sized for
template <int QT, int MT, int EPI, int NT, int WV, int KSW>
__global__ __launch_bounds__(64 * WV, 4 * mb_occ<MT>() / WV) void matvec_batch_kernel(MbJob j, MbTheta<EPI> th) {
    constexpr int THREADS = 64 * WV;
    constexpr int ROWS = 32 * NT;
    constexpr int NCH = mb_nch<QT>();
    constexpr int SB = MbFmt<QT>::SB;
    constexpr int NWI = mb_nwi<QT, NT>();
    constexpr bool XL = mb_xlds<QT, MT>();
    constexpr int NXI = mb_nxi<QT, MT>();
    constexpr int WB = NWI * 1024;
    constexpr int REC = mb_rec(MT);
    constexpr int SLOT = mb_slot<QT, MT, NT>();
    constexpr int NBUF = mb_nbuf<QT, MT>();
    constexpr int XB = mb_xbuf<QT, MT>();
    constexpr int NWL = (NWI + WV - 1) / WV;  // most weight loads of one lane per slab
    constexpr int TPW = NT * KSW / WV;        // tiles per wave
    constexpr int KPW = 16 / KSW;             // k-steps per wave
    constexpr int NXL = XL ? 0 : MT * KPW * 2;  // x register loads of one lane per slab
    static_assert(TPW >= 1 && NT * KSW == TPW * WV && KPW % 2 == 0, "shape");
    static_assert(XL ? NBUF == 1 && XB == 1 : NBUF >= 2 && XB >= 1 && XB <= NBUF, "pipeline depths");
    static_assert(NBUF < 2 || (NBUF - 2) * (NXL + NWL + (NXI + WV - 1) / WV) < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t mb_lds[];

    const int tid = threadIdx.x;
    // wave index in a scalar register (wave-uniform branches)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, h = lane >> 5, col = lane & 31;
    const int kpart = wave / (WV / KSW);
    const int tile0 = (wave % (WV / KSW)) * TPW;
    const int k0 = kpart * KPW;
    const int group = blockIdx.x % j.n_groups;
    const int split = blockIdx.x / j.n_groups;
    const int s0 = split * j.slabs_per_split;
    const int s1 = min(j.n_slabs, s0 + j.slabs_per_split);

    // this lane's weight chunks: instruction wave + WV k covers chunks
    // 64 (wave + WV k) + lane -> (row, chunk)
    const uint8_t* wrow[NWL];
    int wch[NWL];
#pragma unroll
    for (int k = 0; k < NWL; ++k) {
        const int ci = (wave + WV * k) * 64 + lane;
        const int row = ci / NCH;
        wch[k] = row < ROWS ? ci % NCH : 0;
        wrow[k] = mb_row<EPI, ROWS>(j, group, row < ROWS ? row : ROWS - 1);
    }
    // Weights (and Q4_K's x sums) of slab s into LDS slot si: 1 KiB
    // direct-to-LDS instructions dealt round-robin to the waves.
    auto issue_w = [&](int s, int si) {
        uint8_t* slot = mb_lds + si * SLOT;
#pragma unroll
        for (int k = 0; k < NWL; ++k) {
            const int ins = wave + WV * k;
            if (ins >= NWI) break;  // wave-uniform
            if constexpr (SB % 16 == 0) {
                // Q4_0 / Q8_0 / Q4_K: in a 16-byte aligned matrix every slab
                // starts 16-byte aligned, so the lane's chunk of slab s is its
                // chunk of slab 0 plus s * SB (one 64-bit add per load; the
                // general form below costs about nine VALU operations)
                lds_load16(wrow[k] + 16 * wch[k] + (int64_t)s * SB, slot + ins * 1024);
            } else {
                const uintptr_t a = (uintptr_t)(wrow[k] + (int64_t)s * SB);
                const uintptr_t a0 = a & ~(uintptr_t)15;
                const int last = (int)((a + SB - 1 - a0) >> 4);  // last chunk of this row's slab
                const int c = wch[k] < last ? wch[k] : last;
                lds_load16(reinterpret_cast<const void*>(a0 + 16 * (uintptr_t)c), slot + ins * 1024);
            }
        }
        if constexpr (NXI > 0) {
            // the whole record (x through LDS), else its x sums
            const uint8_t* src = j.xrec + (int64_t)s * REC + (XL ? 0 : MT * 32768);
#pragma unroll
            for (int k = 0; k < (NXI + WV - 1) / WV; ++k) {
                const int ins = wave + WV * k;
                if (ins >= NXI) break;
                lds_load16(src + ins * 1024 + 16 * lane, slot + WB + ins * 1024);
            }
        }
    };
    // The wave's x fragments of slab s (its k-steps, hi and lo, every
    // M-tile) into registers: each fragment is 1 KiB of the record, one
    // 16-byte load per lane.
    using XR = mb_h8[MT][KPW][2];
    auto issue_x = [&](int s, XR& xr) {
        if constexpr (XL) return;
        const uint8_t* src = j.xrec + (int64_t)s * REC + lane * 16;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int k = 0; k < KPW; ++k)
#pragma unroll
                for (int hl = 0; hl < 2; ++hl)
                    xr[mt][k][hl] = *reinterpret_cast<const mb_h8*>(
                        src + ((mt * 16 + k0 + k) * 2 + hl) * 1024);
    };

    mb_f16 acc[TPW][MT];
#pragma unroll
    for (int nt = 0; nt < TPW; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.0f;

    // Offset of each of the lane's rows' slab start inside its first 16-byte
    // chunk: the low bits of the row's address, taken once here (the row
    // pointer is picked from the job's matrices with a lane-dependent index,
    // a memory load that inside the loop would wait for every load in flight).
    uint32_t rlow[TPW];
#pragma unroll
    for (int nt = 0; nt < TPW; ++nt)
        rlow[nt] = (uint32_t)(uintptr_t)mb_row<EPI, ROWS>(j, group, (tile0 + nt) * 32 + col) & 15u;

    auto compute = [&](const uint8_t* slot, const XR& xr, int s) {
            // Q4_K: x sums
            const float* meta = reinterpret_cast<const float*>(slot + WB + (XL ? MT * 32768 : 0));
            // x fragment (M-tile mt, the wave's k-step kl, hi or lo)
            auto xfrag = [&](int mt, int kl, int hl) -> mb_h8 {
                if constexpr (XL)
                    return *reinterpret_cast<const mb_h8*>(slot + WB + ((mt * 16 + k0 + kl) * 2 + hl) * 1024 +
                                                           lane * 16);
                else
                    return xr[mt][kl][hl];
            };

            // The wave's tiles one after the other: a tile's block sums are
            // finished and scaled before the next tile's start, so the
            // partial-sum registers are those of one tile (MT chains).
            const uint8_t* rb[TPW];
#pragma unroll
            for (int nt = 0; nt < TPW; ++nt) {
                const int row = (tile0 + nt) * 32 + col;
                rb[nt] = slot + row * NCH * 16 + (int)((rlow[nt] + (uint32_t)s * SB) & 15u);
            }
            // the wave's k-step kl (k0 + kl of the slab): tmp[mt] += A B for
            // the hi and lo halves of A
            auto mfma_step = [&](int kl, const mb_h8& B, mb_f16 (&tmp)[MT]) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    tmp[mt] = mfma(xfrag(mt, kl, 0), B, tmp[mt]);
                    tmp[mt] = mfma(xfrag(mt, kl, 1), B, tmp[mt]);
                }
            };
            auto zero = [&](mb_f16 (&tmp)[MT]) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) tmp[mt][r] = 0.0f;
            };

#pragma unroll
            for (int nt = 0; nt < TPW; ++nt) {
                if constexpr (QT == kQ4_0 || QT == kQ8_0) {
                    constexpr int BB = QT == kQ4_0 ? 18 : 34;
#pragma unroll
                    for (int bi = 0; bi < KPW / 2; ++bi) {
                        const uint8_t* bp = rb[nt] + BB * (k0 / 2 + bi);
                        const float d = h2f((uint16_t)lds_u16(bp));
                        mb_f16 tmp[MT];
                        zero(tmp);
#pragma unroll
                        for (int part = 0; part < 2; ++part) {
                            mb_h8 B;
                            if constexpr (QT == kQ4_0) {
                                B = mb_nibbles(lds_u32(bp + 2 + 8 * part + 4 * h), 0u, -8.0f);
                            } else {
                                const uint8_t* qp = bp + 2 + 16 * part + 8 * h;
                                B = mb_int8(lds_u32(qp), lds_u32(qp + 4));
                            }
                            mfma_step(2 * bi + part, B, tmp);
                        }
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[nt][mt][r] = fmaf(d, tmp[mt][r], acc[nt][mt][r]);
                    }
                } else if constexpr (QT == kQ4_K) {
                    constexpr int NSB = KPW / 2;  // sub-blocks of this wave
                    const float d = h2f((uint16_t)lds_u16(rb[nt]));
                    const float dmin = h2f((uint16_t)lds_u16(rb[nt] + 2));
                    // the wave's sub-blocks' 6-bit scale and minimum (the
                    // q4_K_scale_min packing) from the bytes that hold them:
                    // the sub-block index is wave-uniform, so each is one
                    // byte read rather than a select among the 12 bytes
                    const uint8_t* sb8 = rb[nt] + 4;
                    float mn[NSB];
                    _Float16 f[NSB];
#pragma unroll
                    for (int q = 0; q < NSB; ++q) {
                        const int sb = k0 / 2 + q;
                        int sc, m;
                        if (sb < 4) {
                            sc = sb8[sb] & 0x3F;
                            m = sb8[sb + 4] & 0x3F;
                        } else {
                            const int hi = sb8[sb + 4];
                            sc = ((hi & 0x0F) << 2) | (sb8[sb - 4] >> 6);
                            m = ((hi >> 4) << 2) | (sb8[sb] >> 6);
                        }
                        f[q] = (_Float16)(float)sc;
                        mn[q] = dmin * (float)m;
                    }
                    mb_f16 tmp[MT];
                    zero(tmp);
#pragma unroll
                    for (int k = 0; k < KPW; ++k) {
                        const mb_h8 B = mb_nibbles_scaled(
                            lds_u32(rb[nt] + 16 + 8 * (k0 + k) + 4 * h), f[k >> 1]);  // sc * q <= 945
                        mfma_step(k, B, tmp);
                    }
                    const float* xs = meta + 32 * MT;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int b = mb_token(mt, r, h);
                            float a = fmaf(d, tmp[mt][r], acc[nt][mt][r]);
#pragma unroll
                            for (int q = 0; q < NSB; ++q)
                                a = fmaf(-mn[q], xs[(k0 / 2 + q) * 32 * MT + b], a);
                            acc[nt][mt][r] = a;
                        }
                } else {
                    static_assert(QT == kQ6_K, "format");
                    const float d = h2f((uint16_t)lds_u16(rb[nt] + 208));
#pragma unroll
                    for (int k = 0; k < KPW; ++k) {
                        const int t = k0 + k;
                        const float ds = d * (float)(int8_t)rb[nt][192 + t];
                        const uint32_t hq = lds_u16(rb[nt] + 128 + 4 * t + 2 * h);
                        const uint32_t hs = (hq & 0xFFu) | ((hq & 0xFF00u) << 8);
                        const mb_h8 B = mb_nibbles(lds_u32(rb[nt] + 8 * t + 4 * h), hs, -32.0f);
                        mb_f16 tmp[MT];
                        zero(tmp);
                        mfma_step(k, B, tmp);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[nt][mt][r] = fmaf(ds, tmp[mt][r], acc[nt][mt][r]);
                    }
                }
            }
    };

    // Pipeline: step i (slab s0 + i) waits for its weights and x, passes the
    // workgroup barrier (after which every wave has finished step i - 1, so
    // its slot may be refilled), issues x for step i + XB - 1 and weights for
    // step i + NBUF - 1, then multiplies.  Every step issues the same loads
    // (steps past the last slab re-read the last slab: cache hits, never
    // multiplied), so the wait count is one constant per wave and the
    // compiler's own waits on the x registers see the same loads in flight
    // on every path.  The prologue issues NBUF - 1 steps' loads in the same
    // order (x of steps before 0 re-reads slab s0 into the register set that
    // step XB - 1's load overwrites).
    const int ns = s1 - s0;
    auto clamp = [&](int i) { return s0 + (i < ns ? i : ns - 1); };
    XR xr[XB];
#pragma unroll
    for (int v = -(NBUF - 1); v < 0; ++v) {
        const int xi = v + XB - 1;
        issue_x(clamp(xi < 0 ? 0 : xi), xr[(xi + XB * NBUF) % XB]);
        issue_w(clamp(v + NBUF - 1), (v + NBUF - 1) % NBUF);
    }
    constexpr int U = mb_lcm(NBUF, XB);
    for (int base = 0; base < ns; base += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u;
            if constexpr (NBUF == 1) {
                // one slot: this step's loads, then its product, then a
                // barrier before the next step refills the slot
                issue_w(clamp(i), 0);
                mb_wait_w<NWI, NXI, NXL, NBUF, WV>(wave);
                __syncthreads();
                if (i < ns) compute(mb_lds, xr[0], s0 + i);
                __syncthreads();
            } else {
                mb_wait_w<NWI, NXI, NXL, NBUF, WV>(wave);
                __syncthreads();
                issue_x(clamp(i + XB - 1), xr[(u + XB - 1) % XB]);
                issue_w(clamp(i + NBUF - 1), (u + NBUF - 1) % NBUF);
                if (i < ns) compute(mb_lds + (u % NBUF) * SLOT, xr[u % XB], s0 + i);
            }
        }
    }
    // The reduction below reuses the slots.  The last step's direct-to-LDS
    // loads (a re-read of the last slab) may still be landing there, and a
    // wave's own wait covers only its own loads: every wave waits for its
    // loads before the barrier, so none lands after another wave's writes.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
    __syncthreads();
    // the sums are in units of x * s: 1 / s per token (the same in every
    // slab of the split's records) scales them exactly
    {
        const float* inv = reinterpret_cast<const float*>(j.xrec + (int64_t)s0 * REC + MT * 32768);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float is = inv[mb_token(mt, r, h)];
#pragma unroll
                for (int nt = 0; nt < TPW; ++nt) acc[nt][mt][r] *= is;
            }
    }

    // ---- sum the k-parts (in order) ----
    constexpr int NV = NT * MT * 1024;   // values per workgroup: [tile][mt][r][lane]
    constexpr int PV = NV / THREADS;
    float* red = reinterpret_cast<float*>(mb_lds);
#pragma unroll
    for (int nt = 0; nt < TPW; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                red[(int64_t)kpart * NV + ((tile0 + nt) * MT + mt) * 1024 + r * 64 + lane] =
                    acc[nt][mt][r];
    __syncthreads();
    float val[PV];
#pragma unroll
    for (int i = 0; i < PV; ++i) {
        const int idx = tid + THREADS * i;
        float v = red[idx];
#pragma unroll
        for (int kp = 1; kp < KSW; ++kp) v += red[kp * NV + idx];
        val[i] = v;
    }
    auto token_of = [](int idx) {
        const int mt = (idx >> 10) % MT, r = (idx >> 6) & 15, ln = idx & 63;
        return mb_token(mt, r, ln >> 5);
    };
    auto local_of = [](int idx) { return (idx / (MT * 1024)) * 32 + (idx & 31); };
    if constexpr (EPI == kMbEpiAdd || EPI == kMbEpiQKV) {
        if (j.dpart) {
            // deferred merge: this split's sums go to its own partial array,
            // summed afterwards by a launch of its own (the residual add's
            // merge ahead of the next preparation, the Q / K / V epilogue):
            // no counter, no cross-workgroup merge here
            float* dp = j.dpart + split * j.dstride;
#pragma unroll
            for (int i = 0; i < PV; ++i) {
                const int idx = tid + THREADS * i;
                const int b = token_of(idx);
                const int row = group * ROWS + local_of(idx);
                if (b < j.n_batch && row < j.rows) dp[(int64_t)b * j.rows + row] = val[i];
            }
            return;
        }
    }
    if (j.k_splits > 1) {
        // partials in thread-contiguous order ([group][split][thread][PV]),
        // 16-byte device-coherent (sc1) stores and loads, all loads of the
        // merge issued together
        const int64_t base = ((int64_t)group * j.k_splits) * NV;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            j.part + base, (short)0, j.k_splits * NV * 4, 0x00020000);
        const int off0 = (split * NV + tid * PV) * 4;
#pragma unroll
        for (int i = 0; i < PV; i += 4) {
            const mb_f4 v = {val[i], val[i + 1], val[i + 2], val[i + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(v, rs, off0 + 4 * i, 0, kMbSc1);
        }
        // Every thread waits for its partial stores; the barrier orders them
        // before thread 0's agent-scope release increment of the counter; the
        // workgroup that sees the final count acquires (so it synchronizes
        // with every earlier release) and its threads read the partials after
        // the next barrier.  Only that one workgroup pays the acquire's L2
        // invalidation.  The ordering is the memory model's, not a hardware
        // idiom: it holds whatever the compiler reorders.  (Its cost: a
        // relaxed increment, relying on the partials' device-coherent
        // accesses alone, measured 13 us less over the four batch-32 GEMVs of
        // a layer; acquire-release on every increment 7 us more.)
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        __shared__ int last;
        if (tid == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(j.counters + group, 1u, __ATOMIC_RELEASE,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            last = prev == (uint32_t)(j.k_splits - 1);
            if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (last)
                __hip_atomic_store(j.counters + group, 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        float sum[PV];
#pragma unroll
        for (int i = 0; i < PV; ++i) sum[i] = 0.0f;
        for (int sp = 0; sp < j.k_splits; ++sp) {
            const int off = (sp * NV + tid * PV) * 4;
#pragma unroll
            for (int i = 0; i < PV; i += 4) {
                const mb_f4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * i, 0, kMbSc1);
                sum[i] += v[0];
                sum[i + 1] += v[1];
                sum[i + 2] += v[2];
                sum[i + 3] += v[3];
            }
        }
        // this thread's values in the epilogue order below
#pragma unroll
        for (int i = 0; i < PV; ++i) val[i] = sum[i];
    }

    // ---- epilogue ----
    __syncthreads();  // the reduction area is free again

    if constexpr (EPI == kMbEpiStore || EPI == kMbEpiAdd) {
#pragma unroll
        for (int i = 0; i < PV; ++i) {
            const int idx = tid + THREADS * i;
            const int b = token_of(idx);
            const int row = group * ROWS + local_of(idx);
            if (b < j.n_batch && row < j.rows) {
                float* yp = j.y + (int64_t)b * j.ld_y + row;
                if constexpr (EPI == kMbEpiAdd)
                    *yp = *yp + val[i];
                else
                    *yp = val[i];
            }
        }
    } else if constexpr (EPI == kMbEpiSwiGLU) {
        // gate tiles first: gate value idx < NV / 2, its up value at idx + NV / 2
        static_assert(PV % 2 == 0, "pairs");
#pragma unroll
        for (int i = 0; i < PV / 2; ++i) {
            const int idx = tid + THREADS * i;
            const int b = token_of(idx);
            const int row = group * (ROWS / 2) + local_of(idx);
            if (b < j.n_batch && row < j.rows)
                j.y[(int64_t)b * j.ld_y + row] = swiglu_exact(val[i], val[i + PV / 2]);
        }
    } else {
        // RoPE pairs: rows 2p, 2p + 1 are lanes 2p, 2p + 1 of one register;
        // exchanged through LDS so that each thread holds both halves
        float* pv = reinterpret_cast<float*>(mb_lds);
#pragma unroll
        for (int i = 0; i < PV; ++i) pv[tid + THREADS * i] = val[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PV / 2; ++i) {
            const int idx = 2 * (tid + THREADS * i);  // even lane of the pair
            const int b = token_of(idx);
            const int v0 = group * ROWS + local_of(idx);
            if (b >= j.n_batch || v0 >= j.rows) continue;
            mb_qkv_store(j, th, b, v0, pv[idx], pv[idx + 1]);
        }
    }
}

// ---- host side ----


// A workgroup shape (see above) and what it implies for a matrix.
struct MbShape {
    int nt, wv, ksw;
    int rows_per_group(int epi) const { return epi == kMbEpiSwiGLU ? 16 * nt : 32 * nt; }
};

constexpr MbShape kMbNarrow{2, 4, 4};

// Column splits: as many as keep the workgroups at most kMbSplitTarget
// (rounded down).  Each split adds its partials' device-coherent traffic and
// the merging workgroup's tail; measured at 32 sequences on the Llama-3-8B
// shapes, this count beat rounding up (14336 x 4096: 26.8 against 31.7 us;
// 28672 x 4096: 47.6 against 59.7 us) and smaller targets (4096 x 14336:
// 26.4 us at 512 workgroups, 35.9 at 256).
constexpr int kMbSplitTarget = 512;
// One launch over two M-tiles (more than 32 sequences, every format but
// Q6_K): its 8-wave workgroups take a CU each, so at most 256 of them, one
// round, and fewer partials to merge (Llama-3-8B at batch 64: Q4_0 step 5.48
// -> 5.07 ms, Q4_K_M 7.37 -> 7.14).  Q6_K's two one-tile launches keep the
// common target (at 256: Q4_K_M 7.93 against 7.40 ms).  The sizes reported
// for workspaces and deferred partials use the common target, which gives
// the most splits.
constexpr int kMbSplitTarget2 = 256;
int mb_split_target(int qtype, int n_batch) {
    return n_batch > 32 && qtype != kQ6_K ? kMbSplitTarget2 : kMbSplitTarget;
}
int mb_split(int n_groups, int n_slabs, int* slabs_per_split, int target = kMbSplitTarget) {
    int k = target / n_groups;
    if (k > n_slabs) k = n_slabs;
    if (k < 1) k = 1;
    const int per = (n_slabs + k - 1) / k;
    *slabs_per_split = per;
    return (n_slabs + per - 1) / per;
}

// The 64-row shape for every matrix: measured at 32 sequences on the
// Llama-3-8B step, 8-wave workgroups over 256 (Q4_0) or 128 (Q6_K) rows with
// two LDS slots were slower on the FFN and output matrices (step 5.13 against
// 4.71 ms; 28672 x 4096 alone 56.2 against 44.9 us), and no faster at 8 or 64
// sequences.
MbShape mb_shape() { return kMbNarrow; }

// The counters' area: at least 16 KiB, so that the x records start at the
// same offset for every matrix of up to 4096 row groups (262,144 rows) and one
// preparation can serve several GEMVs of the same input.
size_t mb_ctr_bytes(int n_groups) {
    const size_t b = ((size_t)n_groups * 4 + 255) / 256 * 256;
    return b > 16384 ? b : 16384;
}

// Workspace: the groups' counters, the x records, then the split partials.
size_t mb_ws_bytes(const MbShape& sh, int epi, int out_rows, int n_slabs, int mt) {
    const int groups = (out_rows + sh.rows_per_group(epi) - 1) / sh.rows_per_group(epi);
    int per;
    const int k = mb_split(groups, n_slabs, &per);  // the most splits of any format
    const size_t parts = k > 1 ? (size_t)groups * k * sh.nt * mt * 1024 * 4 : 0;
    return mb_ctr_bytes(groups) + (size_t)n_slabs * mb_rec(mt) + parts;
}

template <int QT, int MT, int EPI, int NT, int WV, int KSW>
int mb_launch_shape(MbJob& j, const MbTheta<EPI>& th, hipStream_t stream) {
    const dim3 grid((unsigned)(j.n_groups * j.k_splits));
    return launch(matvec_batch_kernel<QT, MT, EPI, NT, WV, KSW>, grid, dim3(64 * WV),
                  mb_lds_bytes<QT, MT, NT, KSW>(), stream, j, th);
}

template <int QT, int MT, int EPI>
int mb_launch_t(MbJob& j, const MbShape& sh, const MbTheta<EPI>& th, const void* norm_w,
                int norm_f16, float eps, const MbDefer* pend, hipStream_t stream) {
    const int kg = (j.n_slabs + 7) / 8;  // 8-column groups per thread
    const bool merged = pend && pend->part;
    if (merged) {
        // the pending residual add into x (the residual stream) with the new
        // rows' slice statistics, then the preparation of the completed
        // stream from those statistics
        const int cols = j.n_slabs * kMbCols;
        const int rc = launch(mb_merge_kernel, dim3((unsigned)kg, (unsigned)j.n_batch), dim3(256),
                              0, stream, const_cast<float*>(j.x), j.ld_x, j.n_batch, cols,
                              pend->part, pend->k, pend->stride, norm_w, norm_f16, pend->ss,
                              pend->mx);
        if (rc != JINF_HIP_OK) return rc;
    }
    // without a norm and with split columns: one scale per split's chunk,
    // each preparation workgroup reading only its chunk; after a merge: the
    // 2048-column chunks of the full-row layout, each reading only its own
    const bool chunked = !merged && !norm_w && j.k_splits > 1;
    auto prep = [&](auto kern) {
        return launch(kern, dim3((unsigned)(chunked ? j.k_splits : kg), 32 * MT), dim3(256), 0,
                      stream, j.x, j.ld_x, j.n_batch, j.n_slabs * kMbCols, norm_w, norm_f16, eps,
                      const_cast<uint8_t*>(j.xrec),
                      chunked ? j.slabs_per_split : merged ? kMbSliceCols / kMbCols : 0,
                      merged ? static_cast<const double*>(pend->ss) : nullptr,
                      merged ? static_cast<const float*>(pend->mx) : nullptr, kg);
    };
    const int rc = j.x_ready ? JINF_HIP_OK
                   : merged ? prep(mb_prepare_kernel<MT, 2>)
                   : chunked ? (j.slabs_per_split <= 16   ? prep(mb_prepare_kernel<MT, 2>)
                              : j.slabs_per_split <= 32 ? prep(mb_prepare_kernel<MT, 4>)
                              : j.slabs_per_split <= 64 ? prep(mb_prepare_kernel<MT, 8>)
                                                        : prep(mb_prepare_kernel<MT, 16>))
                   : kg <= 2 ? prep(mb_prepare_kernel<MT, 2>)
                   : kg <= 4 ? prep(mb_prepare_kernel<MT, 4>)
                   : kg <= 8 ? prep(mb_prepare_kernel<MT, 8>)
                             : prep(mb_prepare_kernel<MT, 16>);
    if (rc != JINF_HIP_OK) return rc;
    (void)sh;  // kMbNarrow: 64 rows
    if constexpr (MT == 1)
        return mb_launch_shape<QT, MT, EPI, 2, 4, 4>(j, th, stream);
    else
        return mb_launch_shape<QT, MT, EPI, 2, 8, 8>(j, th, stream);
}

// Sequences 32 .. n_batch - 1 of a job as a job of their own.
template <int EPI>
MbJob mb_upper(const MbJob& j) {
    MbJob u = j;
    u.n_batch = j.n_batch - 32;
    u.x = j.x + (int64_t)32 * j.ld_x;
    u.y = j.y + (int64_t)32 * j.ld_y;
    if (u.dpart) u.dpart += (int64_t)32 * j.rows;
    if constexpr (EPI == kMbEpiQKV) {
        u.pos = j.pos + 32;
        const int64_t es = j.kv_f16 ? 2 : 4;
        if (j.kc) u.kc = static_cast<char*>(j.kc) + 32 * j.ld_seq * es;
        if (j.vc) u.vc = static_cast<char*>(j.vc) + 32 * j.ld_seq * es;
    }
    return u;
}

// More than 32 sequences: one launch over two M-tiles when the shape's LDS
// holds a slot of that size, else two launches of at most 32.
template <int QT, int EPI>
int mb_dispatch_t(MbJob& j, const MbShape& sh, const MbTheta<EPI>& th, const void* norm_w,
                  int norm_f16, float eps, const MbDefer* pend, hipStream_t stream) {
    if (j.n_batch <= 32)
        return mb_launch_t<QT, 1, EPI>(j, sh, th, norm_w, norm_f16, eps, pend, stream);
    // Q6_K at two M-tiles keeps x in LDS (its registers would spill) with one
    // slot, 128 KiB a workgroup: two one-tile launches are faster (the
    // 128256-row output head at 64 sequences: step 5.60 -> 5.56 ms)
    constexpr bool fits = QT != kQ6_K && mb_lds_bytes<QT, 2, 2, 8>() <= 160 * 1024 - 512;  // static LDS aside
    if (fits) return mb_launch_t<QT, 2, EPI>(j, sh, th, norm_w, norm_f16, eps, pend, stream);
    MbJob lo = j;
    lo.n_batch = 32;
    const int rc = mb_launch_t<QT, 1, EPI>(lo, sh, th, norm_w, norm_f16, eps, pend, stream);
    if (rc != JINF_HIP_OK) return rc;
    MbJob hi = mb_upper<EPI>(j);
    MbDefer ph;
    if (pend) {
        ph = *pend;
        if (ph.part) ph.part += (int64_t)32 * j.n_slabs * kMbCols;
    }
    return mb_launch_t<QT, 1, EPI>(hi, sh, th, norm_w, norm_f16, eps, pend ? &ph : nullptr,
                                   stream);
}

template <int EPI>
int mb_dispatch(int qtype, MbJob& j, const MbShape& sh, const MbTheta<EPI>& th,
                const void* norm_w, int norm_f16, float eps, const MbDefer* pend,
                hipStream_t stream) {
    switch (qtype) {
        case kQ4_0: return mb_dispatch_t<kQ4_0, EPI>(j, sh, th, norm_w, norm_f16, eps, pend, stream);
        case kQ8_0: return mb_dispatch_t<kQ8_0, EPI>(j, sh, th, norm_w, norm_f16, eps, pend, stream);
        case kQ4_K: return mb_dispatch_t<kQ4_K, EPI>(j, sh, th, norm_w, norm_f16, eps, pend, stream);
        case kQ6_K: return mb_dispatch_t<kQ6_K, EPI>(j, sh, th, norm_w, norm_f16, eps, pend, stream);
        default: return JINF_HIP_ERR_INVALID;
    }
}

int mb_row_bytes(int qtype, int cols, int64_t* rb) {
    int e, b;
    switch (qtype) {
        case kQ4_0: e = 32; b = 18; break;
        case kQ8_0: e = 32; b = 34; break;
        case kQ4_K: e = 256; b = 144; break;
        case kQ6_K: e = 256; b = 210; break;
        default: return JINF_HIP_ERR_INVALID;
    }
    *rb = (int64_t)(cols / e) * b;
    return JINF_HIP_OK;
}

// Shared checks and job set-up for `rows` output rows of epilogue epi; the
// workgroup shape follows the matrix.
int mb_prepare(MbJob& j, MbShape& sh, int qtype, int epi, int rows, int cols, int n_batch,
               const float* x, int ld_x, float* y, int ld_y, void* ws, size_t ws_bytes) {
    if (rows <= 0 || cols <= 0 || n_batch <= 0 || n_batch > kMbMaxBatch || cols % kMbCols != 0 ||
        cols > kMbMaxCols)
        return JINF_HIP_ERR_INVALID;
    if (!x || !y || !aligned(x, 16) || ld_x % 4 != 0 || ld_x < cols || ld_y <= 0)
        return JINF_HIP_ERR_INVALID;
    if (mb_row_bytes(qtype, cols, &j.row_bytes) != JINF_HIP_OK) return JINF_HIP_ERR_INVALID;
    j.rows = rows;
    j.n_slabs = cols / kMbCols;
    sh = mb_shape();
    j.n_groups = (rows + sh.rows_per_group(epi) - 1) / sh.rows_per_group(epi);
    const int mt = n_batch > 32 ? 2 : 1;
    if (!ws || !aligned(ws, 256) || ws_bytes < mb_ws_bytes(sh, epi, rows, j.n_slabs, mt)) {
        JINF_LOG("batched GEMV: workspace missing, unaligned or smaller than "
                 "jinf_matvec_batch_workspace_bytes()");
        return JINF_HIP_ERR_INVALID;
    }
    j.k_splits =
        mb_split(j.n_groups, j.n_slabs, &j.slabs_per_split, mb_split_target(qtype, n_batch));
    char* w = static_cast<char*>(ws);
    j.counters = reinterpret_cast<uint32_t*>(w);
    j.xrec = reinterpret_cast<uint8_t*>(w + mb_ctr_bytes(j.n_groups));
    j.part = reinterpret_cast<float*>(w + mb_ctr_bytes(j.n_groups) +
                                      (size_t)j.n_slabs * mb_rec(mt));
    j.x = x;
    j.ld_x = ld_x;
    j.n_batch = n_batch;
    j.y = y;
    j.ld_y = ld_y;
    return JINF_HIP_OK;
}

int mb_norm_type(const void* norm_w, int norm_type, float eps, int* f16) {
    if (!norm_w) {
        *f16 = 0;
        return JINF_HIP_OK;
    }
    if ((norm_type != JINF_HIP_F32 && norm_type != JINF_HIP_F16) || !(eps >= 0.0f))
        return JINF_HIP_ERR_INVALID;
    *f16 = norm_type == JINF_HIP_F16;
    return JINF_HIP_OK;
}

bool w_ok(const void* w) { return w && aligned(w, 16); }

}  // namespace

// The largest workspace any epilogue and format can need for this shape.
size_t matvec_batch_ws_bytes(int rows, int cols, int n_batch) {
    if (rows <= 0 || cols <= 0 || cols % kMbCols != 0 || cols > kMbMaxCols || n_batch <= 0 ||
        n_batch > kMbMaxBatch)
        return 0;
    const int mt = n_batch > 32 ? 2 : 1, n_slabs = cols / kMbCols;
    size_t most = 0;
    for (int epi : {kMbEpiStore, kMbEpiSwiGLU}) {
        const size_t b = mb_ws_bytes(mb_shape(), epi, rows, n_slabs, mt);
        most = b > most ? b : most;
    }
    return most;
}

}  // namespace jinf

using namespace jinf;

extern "C" size_t jinf_matvec_batch_workspace_bytes(int rows, int cols, int n_batch) {
    return matvec_batch_ws_bytes(rows, cols, n_batch);
}

extern "C" int jinf_matvec_batch(const void* weight, int qtype, const float* x, int ld_x, float* y,
                                 int ld_y, int rows, int cols, int n_batch, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
    MbJob j{};
    MbShape sh;
    if (!w_ok(weight)) return JINF_HIP_ERR_INVALID;
    const int rc = mb_prepare(j, sh, qtype, kMbEpiStore, rows, cols, n_batch, x, ld_x, y, ld_y,
                              workspace, workspace_bytes);
    if (rc != JINF_HIP_OK) return rc;
    if (ld_y < rows) return JINF_HIP_ERR_INVALID;
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(weight);
    j.seg_end[0] = j.seg_end[1] = j.seg_end[2] = rows;
    return mb_dispatch<kMbEpiStore>(qtype, j, sh, MbNoTheta{}, nullptr, 0, 0.0f, nullptr, stream);
}

extern "C" int jinf_matvec_batch_add(const void* weight, int qtype, const float* x, int ld_x,
                                     float* y, int ld_y, int rows, int cols, int n_batch,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
    MbJob j{};
    MbShape sh;
    if (!w_ok(weight)) return JINF_HIP_ERR_INVALID;
    const int rc = mb_prepare(j, sh, qtype, kMbEpiAdd, rows, cols, n_batch, x, ld_x, y, ld_y,
                              workspace, workspace_bytes);
    if (rc != JINF_HIP_OK) return rc;
    if (ld_y < rows) return JINF_HIP_ERR_INVALID;
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(weight);
    j.seg_end[0] = j.seg_end[1] = j.seg_end[2] = rows;
    return mb_dispatch<kMbEpiAdd>(qtype, j, sh, MbNoTheta{}, nullptr, 0, 0.0f, nullptr, stream);
}

namespace jinf {

int rmsnorm_matvec_batch_m(const void* weight, int qtype, float* h, int ld_h, const void* norm_w,
                           int norm_type, float eps, float* y, int ld_y, int rows, int cols,
                           int n_batch, void* workspace, size_t workspace_bytes,
                           const MbDefer* pend, hipStream_t stream) {
    MbJob j{};
    MbShape sh;
    int f16 = 0;
    if (!w_ok(weight)) return JINF_HIP_ERR_INVALID;
    int rc = mb_prepare(j, sh, qtype, kMbEpiStore, rows, cols, n_batch, h, ld_h, y, ld_y,
                        workspace, workspace_bytes);
    if (rc == JINF_HIP_OK) rc = mb_norm_type(norm_w, norm_type, eps, &f16);
    if (rc != JINF_HIP_OK) return rc;
    if (ld_y < rows) return JINF_HIP_ERR_INVALID;
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(weight);
    j.seg_end[0] = j.seg_end[1] = j.seg_end[2] = rows;
    return mb_dispatch<kMbEpiStore>(qtype, j, sh, MbNoTheta{}, norm_w, f16, eps, pend, stream);
}

int rmsnorm_swiglu_matvec_batch_m(const void* w_gate, const void* w_up, int qtype, float* h,
                                  int ld_h, const void* norm_w, int norm_type, float eps, float* y,
                                  int ld_y, int n_ff, int cols, int n_batch, void* workspace,
                                  size_t workspace_bytes, const MbDefer* pend, hipStream_t stream) {
    MbJob j{};
    MbShape sh;
    int f16 = 0;
    if (!w_ok(w_gate) || !w_ok(w_up)) return JINF_HIP_ERR_INVALID;
    int rc = mb_prepare(j, sh, qtype, kMbEpiSwiGLU, n_ff, cols, n_batch, h, ld_h, y, ld_y,
                        workspace, workspace_bytes);
    if (rc == JINF_HIP_OK) rc = mb_norm_type(norm_w, norm_type, eps, &f16);
    if (rc != JINF_HIP_OK) return rc;
    if (ld_y < n_ff) return JINF_HIP_ERR_INVALID;
    j.W[0] = static_cast<const uint8_t*>(w_gate);
    j.W[1] = static_cast<const uint8_t*>(w_up);
    j.W[2] = j.W[0];
    j.seg_end[0] = j.seg_end[1] = j.seg_end[2] = n_ff;
    return mb_dispatch<kMbEpiSwiGLU>(qtype, j, sh, MbNoTheta{}, norm_w, f16, eps, pend, stream);
}

// rmsnorm_qkv_rope_batch_m; collect (may be null): with split columns the
// deferred job is appended to it, its partials' bytes written to *part_used,
// and no epilogue launched (rmsnorm_qkv_rope_batch_mixed finishes every
// format's job in one launch).
static int qkv_rope_batch(const void* wq, const void* wk, const void* wv, int qtype, float* h,
                          int ld_h, const void* norm_w, int norm_type, float eps, int n_embd,
                          float* q, int ld_q, void* k_cache, void* v_cache, int kv_type,
                          int64_t ld_seq, const int32_t* positions, int max_ctx, int head_dim,
                          int n_heads, int n_heads_kv, float freq_base, int n_batch,
                          void* workspace, size_t workspace_bytes, const MbDefer* pend,
                          float* part, size_t part_bytes, bool x_ready, hipStream_t stream,
                          MbQkvJobs* collect, size_t* part_used) {
    if (part_used) *part_used = 0;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim / 2 > kRopeMaxHalf || n_heads < 0 ||
        n_heads_kv < 0 || !(freq_base > 0.0f) || !positions)
        return JINF_HIP_ERR_INVALID;
    const int qd = wq ? n_heads * head_dim : 0;
    const int kvd = n_heads_kv * head_dim;
    const int rows = qd + (wk ? kvd : 0) + (wv ? kvd : 0);
    if (rows == 0) return JINF_HIP_OK;
    if ((wq && !w_ok(wq)) || (wk && !w_ok(wk)) || (wv && !w_ok(wv))) return JINF_HIP_ERR_INVALID;
    if ((wk && !k_cache) || (wv && !v_cache) || (wq && (!q || ld_q < qd)))
        return JINF_HIP_ERR_INVALID;
    if (kv_type != JINF_HIP_F32 && kv_type != JINF_HIP_F16) return JINF_HIP_ERR_INVALID;
    // ld_seq 0: every row writes into the same cache (the tokens of one
    // prompt, at distinct positions)
    if ((wk || wv) && (max_ctx <= 0 || ld_seq < 0 || (ld_seq != 0 && ld_seq < (int64_t)max_ctx * kvd)))
        return JINF_HIP_ERR_INVALID;
    MbJob j{};
    MbShape sh;
    int f16 = 0;
    float* yq = q ? q : h;
    int rc = mb_prepare(j, sh, qtype, kMbEpiQKV, rows, n_embd, n_batch, h, ld_h, yq,
                        wq ? ld_q : 1, workspace, workspace_bytes);
    if (rc == JINF_HIP_OK) rc = mb_norm_type(norm_w, norm_type, eps, &f16);
    if (rc != JINF_HIP_OK) return rc;
    // segments in q, k, v order; absent matrices take no rows
    const uint8_t* Ws[3] = {static_cast<const uint8_t*>(wq), static_cast<const uint8_t*>(wk),
                            static_cast<const uint8_t*>(wv)};
    const int len[3] = {qd, wk ? kvd : 0, wv ? kvd : 0};
    int end = 0;
    for (int s = 0; s < 3; ++s) {
        end += len[s];
        j.seg_end[s] = end;
        j.W[s] = Ws[s] ? Ws[s] : (Ws[0] ? Ws[0] : Ws[1] ? Ws[1] : Ws[2]);
    }
    j.kc = k_cache;
    j.vc = v_cache;
    j.pos = positions;
    j.kv_f16 = kv_type == JINF_HIP_F16;
    j.kv_dim = kvd;
    j.head_dim = head_dim;
    j.max_ctx = max_ctx;
    j.ld_seq = ld_seq;
    RopeTheta th;
    theta_table(th, head_dim, freq_base);
    // x prepared by the previous call on the same input (records at a fixed
    // workspace offset, whole-row scales); not for Q6_K's two one-tile
    // launches at more than 32 sequences, which prepare per launch
    j.x_ready = x_ready && !(pend && pend->part) && (n_batch <= 32 || qtype != kQ6_K) ? 1 : 0;
    if (part && j.k_splits > 1) {
        // the column splits' merge and the epilogue in a launch of their own
        if (!aligned(part, 16) ||
            part_bytes < (size_t)j.k_splits * n_batch * rows * sizeof(float))
            return JINF_HIP_ERR_INVALID;
        j.dpart = part;
        j.dstride = (int64_t)n_batch * rows;
    }
    rc = mb_dispatch<kMbEpiQKV>(qtype, j, sh, th, norm_w, f16, eps, pend, stream);
    if (rc != JINF_HIP_OK || !j.dpart) return rc;
    const int pairs = n_batch * (rows / 2);
    if (collect) {
        // finished by the caller's one epilogue launch for the layer
        collect->j[collect->n] = j;
        collect->pairs[collect->n] = (collect->n ? collect->pairs[collect->n - 1] : 0) + pairs;
        ++collect->n;
        *part_used = (size_t)j.k_splits * n_batch * rows * sizeof(float);
        return JINF_HIP_OK;
    }
    MbQkvJobs js{};
    js.j[0] = j;
    js.pairs[0] = pairs;
    js.n = 1;
    return launch(mb_qkv_epilogue_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0,
                  stream, js, th);
}

int rmsnorm_qkv_rope_batch_m(const void* wq, const void* wk, const void* wv, int qtype, float* h,
                             int ld_h, const void* norm_w, int norm_type, float eps, int n_embd,
                             float* q, int ld_q, void* k_cache, void* v_cache, int kv_type,
                             int64_t ld_seq, const int32_t* positions, int max_ctx, int head_dim,
                             int n_heads, int n_heads_kv, float freq_base, int n_batch,
                             void* workspace, size_t workspace_bytes, const MbDefer* pend,
                             float* part, size_t part_bytes, bool x_ready, hipStream_t stream) {
    return qkv_rope_batch(wq, wk, wv, qtype, h, ld_h, norm_w, norm_type, eps, n_embd, q, ld_q,
                          k_cache, v_cache, kv_type, ld_seq, positions, max_ctx, head_dim,
                          n_heads, n_heads_kv, freq_base, n_batch, workspace, workspace_bytes,
                          pend, part, part_bytes, x_ready, stream, nullptr, nullptr);
}

// Partials region of one format group's deferred Q / K / V launch: 256-byte
// aligned, so that the next group's partials start 16-byte aligned.
static size_t mb_qkv_part_span(size_t used) { return (used + 255) / 256 * 256; }

int rmsnorm_qkv_rope_batch_mixed(const void* const w[3], const int types[3], float* h, int ld_h,
                                 const void* norm_w, int norm_type, float eps, int n_embd,
                                 float* q, int ld_q, void* k_cache, void* v_cache, int kv_type,
                                 int64_t ld_seq, const int32_t* positions, int max_ctx,
                                 int head_dim, int n_heads, int n_heads_kv, float freq_base,
                                 int n_batch, void* workspace, size_t workspace_bytes,
                                 const MbDefer* pend, float* part, size_t part_bytes,
                                 hipStream_t stream) {
    bool done[3] = {false, false, false};
    MbQkvJobs js{};
    const MbDefer* pd = pend;
    // x prepared by an earlier call in the one-launch record layout (Q6_K
    // beyond 32 rows runs two one-tile launches, each preparing its own)
    bool prepared = false;
    size_t off = 0;
    for (int i = 0; i < 3; ++i) {
        if (done[i]) continue;
        const void* p[3] = {nullptr, nullptr, nullptr};
        for (int k = i; k < 3; ++k)
            if (!done[k] && types[k] == types[i]) {
                p[k] = w[k];
                done[k] = true;
            }
        size_t used = 0;
        const int rc = qkv_rope_batch(
            p[0], p[1], p[2], types[i], h, ld_h, norm_w, norm_type, eps, n_embd, q, ld_q,
            k_cache, v_cache, kv_type, ld_seq, positions, max_ctx, head_dim, n_heads, n_heads_kv,
            freq_base, n_batch, workspace, workspace_bytes, pd,
            part ? reinterpret_cast<float*>(reinterpret_cast<char*>(part) + off) : nullptr,
            part_bytes > off ? part_bytes - off : 0, prepared, stream, &js, &used);
        if (rc != JINF_HIP_OK) return rc;
        off += mb_qkv_part_span(used);
        pd = nullptr;
        prepared = n_batch <= 32 || types[i] != kQ6_K;
    }
    if (js.n == 0) return JINF_HIP_OK;
    RopeTheta th;
    theta_table(th, head_dim, freq_base);
    const int pairs = js.pairs[js.n - 1];
    return launch(mb_qkv_epilogue_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0,
                  stream, js, th);
}

size_t qkv_defer_bytes(const int types[3], int q_dim, int kv_dim, int n_embd, int n_batch) {
    const int dims[3] = {q_dim, kv_dim, kv_dim};
    bool done[3] = {false, false, false};
    size_t total = 0;
    for (int i = 0; i < 3; ++i) {
        if (done[i]) continue;
        int rows = 0;
        for (int k = i; k < 3; ++k)
            if (!done[k] && types[k] == types[i]) {
                rows += dims[k];
                done[k] = true;
            }
        // (matvec_batch_defer_bytes counts the same 64-row groups and splits)
        total += mb_qkv_part_span(matvec_batch_defer_bytes(rows, n_embd, n_batch));
    }
    return total;
}

uint8_t* matvec_batch_add_xrec(void* workspace, int qtype, int rows, int cols, int n_batch,
                               int* chunk_cols) {
    *chunk_cols = 0;
    if (!workspace || rows <= 0 || cols <= 0 || cols % kMbCols != 0 || cols > kMbMaxCols ||
        n_batch <= 0 || n_batch > kMbMaxBatch)
        return nullptr;
    const MbShape sh = mb_shape();
    const int groups = (rows + sh.rows_per_group(kMbEpiAdd) - 1) / sh.rows_per_group(kMbEpiAdd);
    int per;
    const int k = mb_split(groups, cols / kMbCols, &per, mb_split_target(qtype, n_batch));
    // (Q6_K at two M-tiles runs as two one-tile launches, each preparing its own)
    if (k > 1 && (cols / kMbCols) % per == 0 && (n_batch <= 32 || qtype != kQ6_K))
        *chunk_cols = per * kMbCols;
    return static_cast<uint8_t*>(workspace) + mb_ctr_bytes(groups);
}

size_t matvec_batch_defer_bytes(int rows, int cols, int n_batch) {
    if (rows <= 0 || cols <= 0 || cols % kMbCols != 0 || cols > kMbMaxCols || n_batch <= 0 ||
        n_batch > kMbMaxBatch)
        return 0;
    const MbShape sh = mb_shape();
    const int groups = (rows + sh.rows_per_group(kMbEpiAdd) - 1) / sh.rows_per_group(kMbEpiAdd);
    int per;
    const int k = mb_split(groups, cols / kMbCols, &per);  // the most splits of any format
    // the partials, then the merge's slice statistics (fp64 sums, fp32 maxima)
    const size_t slices = (size_t)(rows + kMbSliceCols - 1) / kMbSliceCols;
    return (size_t)k * n_batch * rows * sizeof(float) + slices * n_batch * (8 + 4);
}

int matvec_batch_add_defer(const void* weight, int qtype, const float* x, int ld_x, int rows,
                           int cols, int n_batch, float* part, size_t part_bytes, void* workspace,
                           size_t workspace_bytes, MbDefer* out, bool x_ready, hipStream_t stream) {
    MbJob j{};
    MbShape sh;
    if (!w_ok(weight) || !out || !part || !aligned(part, 16)) return JINF_HIP_ERR_INVALID;
    const int rc = mb_prepare(j, sh, qtype, kMbEpiAdd, rows, cols, n_batch, x, ld_x, part, rows,
                              workspace, workspace_bytes);
    if (rc != JINF_HIP_OK) return rc;
    if (part_bytes < matvec_batch_defer_bytes(rows, cols, n_batch)) return JINF_HIP_ERR_INVALID;
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(weight);
    j.seg_end[0] = j.seg_end[1] = j.seg_end[2] = rows;
    j.dpart = part;
    j.dstride = (int64_t)n_batch * rows;
    // records written by the producer: only where the preparation would be
    // chunked the same way (no norm, split columns) and one launch covers
    // every sequence (two M-tiles fit)
    j.x_ready = x_ready && j.k_splits > 1 && (n_batch <= 32 || qtype != kQ6_K) ? 1 : 0;
    out->part = part;
    out->k = j.k_splits;
    out->stride = j.dstride;
    const int64_t slices = (rows + kMbSliceCols - 1) / kMbSliceCols;
    out->ss = reinterpret_cast<double*>(part + (int64_t)j.k_splits * j.dstride);
    out->mx = reinterpret_cast<float*>(out->ss + slices * n_batch);
    return mb_dispatch<kMbEpiAdd>(qtype, j, sh, MbNoTheta{}, nullptr, 0, 0.0f, nullptr, stream);
}

}  // namespace jinf

extern "C" int jinf_rmsnorm_matvec_batch(const void* weight, int qtype, const float* h, int ld_h,
                                         const void* norm_w, int norm_type, float eps, float* y,
                                         int ld_y, int rows, int cols, int n_batch,
                                         void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
    return rmsnorm_matvec_batch_m(weight, qtype, const_cast<float*>(h), ld_h, norm_w, norm_type,
                                  eps, y, ld_y, rows, cols, n_batch, workspace, workspace_bytes,
                                  nullptr, stream);
}

extern "C" int jinf_rmsnorm_swiglu_matvec_batch(const void* w_gate, const void* w_up, int qtype,
                                                const float* h, int ld_h, const void* norm_w,
                                                int norm_type, float eps, float* y, int ld_y,
                                                int n_ff, int cols, int n_batch, void* workspace,
                                                size_t workspace_bytes, hipStream_t stream) {
    return rmsnorm_swiglu_matvec_batch_m(w_gate, w_up, qtype, const_cast<float*>(h), ld_h, norm_w,
                                         norm_type, eps, y, ld_y, n_ff, cols, n_batch, workspace,
                                         workspace_bytes, nullptr, stream);
}

extern "C" int jinf_rmsnorm_qkv_rope_batch(const void* wq, const void* wk, const void* wv,
                                           int qtype, const float* h, int ld_h,
                                           const void* norm_w, int norm_type, float eps,
                                           int n_embd, float* q, int ld_q, void* k_cache,
                                           void* v_cache, int kv_type, int64_t ld_seq,
                                           const int32_t* positions, int max_ctx, int head_dim,
                                           int n_heads, int n_heads_kv, float freq_base,
                                           int n_batch, void* workspace, size_t workspace_bytes,
                                           hipStream_t stream) {
    return rmsnorm_qkv_rope_batch_m(wq, wk, wv, qtype, const_cast<float*>(h), ld_h, norm_w,
                                    norm_type, eps, n_embd, q, ld_q, k_cache, v_cache, kv_type,
                                    ld_seq, positions, max_ctx, head_dim, n_heads, n_heads_kv,
                                    freq_base, n_batch, workspace, workspace_bytes, nullptr,
                                    nullptr, 0, false, stream);
}
