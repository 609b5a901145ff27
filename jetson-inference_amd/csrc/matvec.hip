// Dequant + matrix-vector product for gfx950, for every weight format the
// reference's jinf_cuda_dequant_matvec serves: Q4_0, Q8_0, Q4_K, Q6_K.
//
// Semantics (reference cuda/matmul_kernels.cu:8-185 and the launcher
// :198-225): W is [rows, cols] stored as GGUF blocks along the columns
// (include/jinf/quant.h:30-68, jinf's element orders);
//   y[row] = sum_j w(row, j) * x[j]
// in fp32, with w the reference's dequantized weight.  The summation order is
// not the reference's (its per-thread strided loop and warp tree); results
// agree to the fp32 rounding of the dot product.
//
// Design: batch-1 decode is HBM-bound on the weight bytes (0.5625 B per
// weight for Q4_0 and Q4_K, 0.82 for Q6_K, 1.06 for Q8_0), so every weight
// byte is read once, with nontemporal coalesced 16-byte loads, and x is kept
// out of the per-row traffic:
//   - a column tile is 4096 values of a row (2304 B for Q4_0 / Q4_K, 3360 B
//     for Q6_K, 4352 B for Q8_0); lane l owns values 64 l .. 64 l + 63 of it;
//   - a work item is R rows x one tile; a wave owns whole groups of R rows and
//     walks their tiles, prefetching the next item's bytes into registers
//     while it computes the current one;
//   - the tile bytes go through the wave's own LDS region, where each lane
//     reads back the bytes of its 64 values;
//   - x is staged once per workgroup in LDS; a lane keeps its 64 x values in
//     registers (for the whole kernel when the matrix is one tile wide) and
//     reuses them for all R rows;
//   - dequantisation is folded into the dot product: the integer codes are
//     multiplied as fp16 denormals with v_fma_mix_f32 (see mix2), and the
//     per-block scale, offset and minimum are applied once per block or
//     sub-block against the block's sum of x;
//   - each row's lane partials meet in a DPP wave reduction.
// Anything the tiled kernel does not serve (unaligned pointers, widths that
// are not a multiple of the format's tile granule, more than 7 tiles) takes a
// one-wave-per-row kernel that decodes every weight exactly (quant_device.h).
#include "jinf_device.h"
#include "jinf_host.h"
#include "quant_device.h"
#include "jinf/kernels.h"
#include "jinf/kernels_ext.h"

namespace jinf {

constexpr int kMvTileElems = 4096;                // values of a row per column tile
constexpr int kMvLaneElems = kMvTileElems / kWave;  // 64 values per lane
constexpr int kMvMaxTiles = 7;                    // x of 7 tiles (112 KiB) fits in LDS

// ---- fp16-denormal products ----
//
// Masking a word so that each 16-bit half keeps one small unsigned code c
// (c < 1024) leaves two halves whose bits ARE the fp16 values c * 2^-24,
// exactly.  v_fma_mix_f32 widens such a half and accumulates (c * 2^-24) * x
// in fp32 with a single rounding: one VALU op per weight.  A code stored at
// bit 4 of its half is 16 c: the caller divides the matching x by 16 (exact)
// instead.  The 2^-24 is given back to the block scale (exact).
typedef _Float16 mv_half2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float mix2(uint32_t h, float xlo, float xhi, float acc) {
    const mv_half2 v = __builtin_bit_cast(mv_half2, h);
    acc = fmaf((float)v.x, xlo, acc);
    return fmaf((float)v.y, xhi, acc);
}

constexpr float kTwo24 = 16777216.0f;         // 2^24
constexpr float kTwoM24 = 1.0f / 16777216.0f;  // 2^-24

// 2^-24 * sum_j q_j x_j over 32 values whose 4-bit codes q (0..15) are packed
// in jinf's interleaved order: word i holds values 8i..8i+7, value 8i+n in
// bits 4n..4n+3.  xp: the 32 x values with odd positions pre-divided by 16.
//   w & 0x000F000F        -> values 8i+0 (lo half), 8i+4 (hi half)
//   w & 0x00F000F0        -> 8i+1, 8i+5 (codes times 16)
//   (w >> 8) & 0x000F000F -> 8i+2, 8i+6
//   (w >> 8) & 0x00F000F0 -> 8i+3, 8i+7 (codes times 16)
__device__ __forceinline__ float nib_dot32(const uint32_t (&qw)[4], const float* xp) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = qw[i];
        const uint32_t v = w >> 8;
        const float* xi = xp + 8 * i;
        s = mix2(w & 0x000F000Fu, xi[0], xi[4], s);
        s = mix2(w & 0x00F000F0u, xi[1], xi[5], s);
        s = mix2(v & 0x000F000Fu, xi[2], xi[6], s);
        s = mix2(v & 0x00F000F0u, xi[3], xi[7], s);
    }
    return s;
}

// Same for 8-bit codes (0..255), four per word in value order: word i holds
// values 4i..4i+3 as bytes.
__device__ __forceinline__ float byte_dot(const uint32_t* qw, int nw, const float* x) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < nw; ++i) {
        const uint32_t w = qw[i];
        s = mix2(w & 0x00FF00FFu, x[4 * i], x[4 * i + 2], s);
        s = mix2((w >> 8) & 0x00FF00FFu, x[4 * i + 1], x[4 * i + 3], s);
    }
    return s;
}

// Dword view of LDS bytes at any 2-byte-aligned offset: two aligned reads and
// a funnel shift (shift 0 returns the first word).
__device__ __forceinline__ uint32_t lds_dw(const uint32_t* base, int byte_off) {
    const int k = byte_off >> 2;
    return __builtin_amdgcn_alignbit(base[k + 1], base[k], (byte_off & 3) * 8);
}

// ---- format policies for the tiled kernel ----
//
// Each gives the block geometry, the width granule of the fast path (a
// multiple that makes row and tile byte counts multiples of 16), the rows per
// item, how a lane's x registers are prepared, and the lane's dot product over
// its 64 values of one staged row tile (`row`: the tile's bytes in LDS as
// dwords; xs[k]: plain sum of the lane's x values 16k .. 16k+15).

template <int QT> struct MvFmt;

// Q4_0: lane = 2 consecutive blocks (36 B, 9 dwords at 9 * lane: conflict
// free).  y += d * (2^24 * nib_dot - 8 * sum x) per block, with the 2^24 in d.
template <> struct MvFmt<kQ4_0> {
    static constexpr int kElems = 32, kBytes = 18, kColGranule = 256, kRows = 2;
    static __device__ void prep(float (&xv)[64]) {
#pragma unroll
        for (int i = 1; i < 64; i += 2) xv[i] *= 0.0625f;
    }
    static __device__ float dot(const uint32_t* row, int lane, const float (&xv)[64],
                                const float (&xs)[4]) {
        const uint32_t* l = row + 9 * lane;
        uint32_t D[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) D[i] = l[i];
        const float d0 = h2f((uint16_t)(D[0] & 0xFFFFu)) * kTwo24;
        const float d1 = h2f((uint16_t)(D[4] >> 16)) * kTwo24;
        const uint32_t q0[4] = {__builtin_amdgcn_alignbit(D[1], D[0], 16),
                                __builtin_amdgcn_alignbit(D[2], D[1], 16),
                                __builtin_amdgcn_alignbit(D[3], D[2], 16),
                                __builtin_amdgcn_alignbit(D[4], D[3], 16)};
        const uint32_t q1[4] = {D[5], D[6], D[7], D[8]};
        const float s0 = fmaf(-8.0f * kTwoM24, xs[0] + xs[1], nib_dot32(q0, xv));
        const float s1 = fmaf(-8.0f * kTwoM24, xs[2] + xs[3], nib_dot32(q1, xv + 32));
        return fmaf(d1, s1, d0 * s0);
    }
};

// Q8_0: lane = 2 consecutive blocks (68 B, 17 dwords at 17 * lane: conflict
// free).  The int8 codes are biased to unsigned (q ^ 0x80 = q + 128) for the
// fp16-denormal product, and the bias comes back as -128 * sum x per block.
template <> struct MvFmt<kQ8_0> {
    static constexpr int kElems = 32, kBytes = 34, kColGranule = 256, kRows = 1;
    static __device__ void prep(float (&)[64]) {}
    static __device__ float dot(const uint32_t* row, int lane, const float (&xv)[64],
                                const float (&xs)[4]) {
        const uint32_t* l = row + 17 * lane;
        uint32_t D[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) D[i] = l[i];
        const float d0 = h2f((uint16_t)(D[0] & 0xFFFFu)) * kTwo24;
        const float d1 = h2f((uint16_t)(D[8] >> 16)) * kTwo24;
        uint32_t q0[8], q1[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            q0[i] = __builtin_amdgcn_alignbit(D[i + 1], D[i], 16) ^ 0x80808080u;
            q1[i] = D[9 + i] ^ 0x80808080u;
        }
        const float s0 = fmaf(-128.0f * kTwoM24, xs[0] + xs[1], byte_dot(q0, 8, xv));
        const float s1 = fmaf(-128.0f * kTwoM24, xs[2] + xs[3], byte_dot(q1, 8, xv + 32));
        return fmaf(d1, s1, d0 * s0);
    }
};

// Q4_K: lane = one quarter of a super-block (sub-blocks 2k, 2k+1 of block
// lane / 4, k = lane % 4): header dwords 0-3 of the block (shared by its four
// lanes) and 8 dwords of nibbles.  Per sub-block:
//   sum_j (sub_d q_j - sub_min) x_j = sub_d * sum q x - sub_min * sum x.
template <> struct MvFmt<kQ4_K> {
    static constexpr int kElems = 256, kBytes = 144, kColGranule = 256, kRows = 2;
    static __device__ void prep(float (&xv)[64]) {
#pragma unroll
        for (int i = 1; i < 64; i += 2) xv[i] *= 0.0625f;
    }
    static __device__ float dot(const uint32_t* row, int lane, const float (&xv)[64],
                                const float (&xs)[4]) {
        const int k = lane & 3;
        const uint32_t* b = row + 36 * (lane >> 2);
        const uint32_t h = b[0];
        const uint32_t s[3] = {b[1], b[2], b[3]};
        uint32_t q0[4], q1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q0[i] = b[4 + 8 * k + i];
            q1[i] = b[8 + 8 * k + i];
        }
        const float d = h2f((uint16_t)(h & 0xFFFFu)) * kTwo24;
        const float dmin = h2f((uint16_t)(h >> 16));
        int sc0, mn0, sc1, mn1;
        q4_K_scale_min(s, 2 * k, sc0, mn0);
        q4_K_scale_min(s, 2 * k + 1, sc1, mn1);
        const float t0 = fmaf(d * (float)sc0, nib_dot32(q0, xv), -(dmin * (float)mn0) * (xs[0] + xs[1]));
        const float t1 = fmaf(d * (float)sc1, nib_dot32(q1, xv + 32), -(dmin * (float)mn1) * (xs[2] + xs[3]));
        return t0 + t1;
    }
};

// Q6_K: lane = one quarter of a super-block (values 64k .. 64k+63 of block
// lane / 4): 32 bytes of ql, 16 of qh, 4 int8 scales and d.  Blocks are
// 210 B, so odd blocks start 2 bytes off a dword and are read through lds_dw.
// Per 8 values (one ql word, two qh bytes h0 h1) the 6-bit codes are built as
// bytes in two words, even values and odd values:
//   P  = [h0, h0, h1, h1]
//   Lq = (ql & 0x0F0F0F0F)      | (P << 4 & 0x00300030) | (P & 0x30003000)
//   Hq = (ql >> 4 & 0x0F0F0F0F) | (P << 2 & 0x00300030) | (P >> 2 & 0x30003000)
// (value 2m gets bits 4m'..4m'+1 of its qh byte at bits 4-5 of its byte; see
// the reference's low4 | high2 << 4, cuda/matmul_kernels.cu:164-172).
// Per 16-value sub-block: (d * scale) * (sum q6 x - 32 sum x).
template <> struct MvFmt<kQ6_K> {
    static constexpr int kElems = 256, kBytes = 210, kColGranule = 2048, kRows = 1;
    static __device__ void prep(float (&)[64]) {}
    static __device__ float dot(const uint32_t* row, int lane, const float (&xv)[64],
                                const float (&xs)[4]) {
        const int k = lane & 3;
        const int base = 210 * (lane >> 2);
        uint32_t ql[8], qh[4];
#pragma unroll
        for (int i = 0; i < 8; ++i) ql[i] = lds_dw(row, base + 32 * k + 4 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) qh[i] = lds_dw(row, base + 128 + 16 * k + 4 * i);
        const uint32_t sc = lds_dw(row, base + 192 + 4 * k);
        const float d = h2f((uint16_t)(lds_dw(row, base + 208) & 0xFFFFu)) * kTwo24;
        float acc = 0.0f;
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
            float s = 0.0f;
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
                const int g = 2 * sub + gg;  // 8-value group within the lane
                const uint32_t P = __builtin_amdgcn_perm(0u, qh[g >> 1],
                                                         (g & 1) ? 0x03030202u : 0x01010000u);
                const uint32_t w = ql[g];
                const uint32_t Lq = (w & 0x0F0F0F0Fu) | ((P << 4) & 0x00300030u) | (P & 0x30003000u);
                const uint32_t Hq = ((w >> 4) & 0x0F0F0F0Fu) | ((P << 2) & 0x00300030u) |
                                    ((P >> 2) & 0x30003000u);
                const float* x8 = xv + 8 * g;
                // Lq bytes: values 0, 2, 4, 6 of the group; Hq: 1, 3, 5, 7
                s = mix2(Lq & 0x00FF00FFu, x8[0], x8[4], s);
                s = mix2((Lq >> 8) & 0x00FF00FFu, x8[2], x8[6], s);
                s = mix2(Hq & 0x00FF00FFu, x8[1], x8[5], s);
                s = mix2((Hq >> 8) & 0x00FF00FFu, x8[3], x8[7], s);
            }
            const float scale = d * (float)(int8_t)((sc >> (8 * sub)) & 0xFFu);
            acc = fmaf(scale, fmaf(-32.0f * kTwoM24, xs[sub], s), acc);
        }
        return acc;
    }
};

template <int QT> struct MvTile {
    using F = MvFmt<QT>;
    static constexpr int kTileBlocks = kMvTileElems / F::kElems;
    static constexpr int kTileBytes = kTileBlocks * F::kBytes;
    static constexpr int kChunks = kTileBytes / 16;
    static constexpr int kCPL = (kChunks + kWave - 1) / kWave;  // 16-byte chunks per lane
    // chunk slots past a row's kChunks that the last pass writes (see stage)
    static constexpr int kPad = kWave * kCPL - kChunks;
    static constexpr int kStageChunks = F::kRows * kChunks + kPad;  // per wave
    static_assert(kTileBytes % 16 == 0, "tile must be whole 16-byte chunks");
    static_assert(kPad < kWave, "pad must be rewritten by the first pass");
};

// x tile layout in LDS: tile t holds 1024 float4 (4096 floats); lane l's 16
// float4 sit in row l with the column XOR-swizzled by l & 15, so the 16 lanes
// of one LDS pass read 16 distinct bank groups.
__device__ __forceinline__ int mv_xslot(int tile, int l, int j) {
    return (tile << 10) + (l << 4) + (j ^ (l & 15));
}

// Each wave takes whole groups of R rows (groups g, g + stride, ...) and
// walks their tiles in order, so a row's partial sums stay in registers until
// its last tile.  The wave's LDS accesses execute in order; the fences keep
// the compiler from moving the read-back above the stores.  The only
// workgroup barrier follows the x staging.
template <int QT, bool ONE_TILE>
__global__ __launch_bounds__(ONE_TILE ? 256 : 512) void matvec_kernel(
    const uint8_t* __restrict__ W, int64_t row_bytes, const float* __restrict__ x,
    float* __restrict__ y, int rows, int nb, int nt) {
    using F = MvFmt<QT>;
    using T = MvTile<QT>;
    constexpr int R = F::kRows;
    constexpr int CPL = T::kCPL;
    extern __shared__ uint4 lds[];
    float4* xl = reinterpret_cast<float4*>(lds);
    const int waves = blockDim.x / kWave;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    uint4* stage = lds + (nt << 10) + wave * T::kStageChunks;
    const int n_groups = (rows + R - 1) / R;
    const int stride = gridDim.x * waves;
    if (ONE_TILE) nt = 1;

    using Buf = uint4[R][CPL];
    auto fetch = [&](int g, int t, Buf& buf) {
        const int tb = t * T::kTileBlocks;
        const int nbt = nb - tb < T::kTileBlocks ? nb - tb : T::kTileBlocks;
        const int nchunk = nbt * F::kBytes / 16;  // whole by the width granule
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = g * R + r < rows ? g * R + r : rows - 1;
            const uint8_t* src = W + (int64_t)row * row_bytes + (int64_t)tb * F::kBytes;
#pragma unroll
            for (int k = 0; k < CPL; ++k) {
                // Lanes past the tile's end re-read its last chunk (never used).
                const int c = lane + kWave * k < nchunk ? lane + kWave * k : nchunk - 1;
                buf[r][k] = ld16<true>(src + 16 * c);
            }
        }
    };
    auto advance = [&](int& g, int& t) {
        if (ONE_TILE) {
            g += stride;
        } else if (++t == nt) {
            t = 0;
            g += stride;
        }
    };

    int g0 = blockIdx.x * waves + wave, t0 = 0;
    uint4 bufA[R][CPL];
    uint4 bufB[R][CPL];
    if (g0 < n_groups) fetch(g0, t0, bufA);

    // Stage x (zero past the last value) while the first weights are in flight.
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (int f = threadIdx.x; f < (nt << 10); f += blockDim.x) {
        const float4 v = f < nb * (F::kElems / 4) ? x4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
        xl[mv_xslot(f >> 10, (f >> 4) & 63, f & 15)] = v;
    }
    __syncthreads();
    if (g0 >= n_groups) return;

    float xv[kMvLaneElems];
    float xs[4];
    auto load_x = [&](int t) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float4 v = xl[mv_xslot(t, lane, j)];
            xv[4 * j] = v.x; xv[4 * j + 1] = v.y; xv[4 * j + 2] = v.z; xv[4 * j + 3] = v.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) s += xv[16 * k + i];
            xs[k] = s;
        }
        F::prep(xv);
    };
    if (ONE_TILE) load_x(0);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    auto process = [&](int g, int t, const Buf& buf) {
        if (!ONE_TILE) load_x(t);
        const bool live = t * kMvTileElems + lane * kMvLaneElems < nb * F::kElems;
        // Every lane writes every chunk (no branch, so no load is left pending
        // on a skipped path).  The last pass goes first: its slots past
        // kChunks land on the next row's first chunks, which the first pass
        // then overwrites (a wave's LDS writes complete in order), and the
        // last row's on the pad.
#pragma unroll
        for (int r = 0; r < R; ++r) stage[r * T::kChunks + lane + (CPL - 1) * kWave] = buf[r][CPL - 1];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < CPL - 1; ++k) stage[r * T::kChunks + lane + kWave * k] = buf[r][k];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t* rowp = reinterpret_cast<const uint32_t*>(stage + r * T::kChunks);
            if (live) acc[r] += F::dot(rowp, lane, xv, xs);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (t == nt - 1) {  // group complete: reduce and store its rows
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v = wave_sum_f32(acc[r]);
                if (lane == 0 && g * R + r < rows) y[g * R + r] = v;
                acc[r] = 0.0f;
            }
        }
    };

    // The last item leaves through its own branch, so on the main path the
    // prefetch is unconditional and the compiler's wait counts stay exact
    // (a conditional load makes it wait for every outstanding load).
    int g1 = g0, t1 = t0;
    while (true) {
        advance(g1, t1);
        if (g1 >= n_groups) {
            process(g0, t0, bufA);
            break;
        }
        fetch(g1, t1, bufB);
        process(g0, t0, bufA);
        g0 = g1;
        t0 = t1;
        advance(g1, t1);
        if (g1 >= n_groups) {
            process(g0, t0, bufB);
            break;
        }
        fetch(g1, t1, bufA);
        process(g0, t0, bufB);
        g0 = g1;
        t0 = t1;
    }
}

// Any width / alignment: one wave per row; each lane takes 8-value groups
// with stride 64 and decodes them exactly (byte loads), then fma with x.
template <int QT>
__global__ __launch_bounds__(256) void matvec_any_kernel(const uint8_t* __restrict__ W,
                                                         int64_t row_bytes,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int rows, int nb) {
    constexpr int E = QGeom<QT>::kElems, B = QGeom<QT>::kBytes;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const uint8_t* wr = W + row * row_bytes;
    const int n_groups = nb * (E / 8);
    float acc = 0.0f;
    for (int gi = lane; gi < n_groups; gi += kWave) {
        const int b = gi / (E / 8);
        const int e0 = (gi % (E / 8)) * 8;
        float w[8];
        decode8<QT>(wr + (int64_t)b * B, e0, w);
        const float* xp = x + (int64_t)8 * gi;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(w[i], xp[i], acc);
    }
    acc = wave_sum_f32(acc);
    if (lane == 0) y[row] = acc;
}

// Launch the tiled kernel with at most grid_cap workgroups.  Single-tile
// matrices use 4 independent waves per workgroup; wider ones 8 waves sharing
// one copy of x.  Returns JINF_HIP_ERR_INVALID when the shape is not served.
template <int QT>
static int mv_launch(const void* w, const float* x, float* y, int rows, int cols, int grid_cap,
                     hipStream_t stream) {
    using F = MvFmt<QT>;
    using T = MvTile<QT>;
    if (cols % F::kColGranule != 0) return JINF_HIP_ERR_INVALID;
    const int nb = cols / F::kElems;
    const int nt = (cols + kMvTileElems - 1) / kMvTileElems;
    if (nt > kMvMaxTiles) return JINF_HIP_ERR_INVALID;
    const int waves = nt == 1 ? 4 : 8;
    const int groups = (rows + F::kRows - 1) / F::kRows;
    int grid = (groups + waves - 1) / waves;
    if (grid > grid_cap) grid = grid_cap;
    const size_t shmem = ((size_t)nt * 1024 + (size_t)waves * T::kStageChunks) * 16;
    const uint8_t* W = static_cast<const uint8_t*>(w);
    const int64_t row_bytes = (int64_t)nb * F::kBytes;
    if (nt == 1)
        return launch(matvec_kernel<QT, true>, dim3(grid), dim3(waves * kWave), shmem, stream, W,
                      row_bytes, x, y, rows, nb, nt);
    return launch(matvec_kernel<QT, false>, dim3(grid), dim3(waves * kWave), shmem, stream, W,
                  row_bytes, x, y, rows, nb, nt);
}

template <int QT>
static int matvec_t(const void* w, const float* x, float* y, int rows, int cols,
                    hipStream_t stream) {
    using F = MvFmt<QT>;
    const int nb = cols / F::kElems;
    if (cols % F::kColGranule == 0 && cols <= kMvMaxTiles * kMvTileElems && aligned(w, 16) &&
        aligned(x, 16)) {
        // 512 workgroups (two per CU on 256 CUs) measured best for Q4_0 at
        // 4096-14336 rows; each wave then streams several items.
        return mv_launch<QT>(w, x, y, rows, cols, 512, stream);
    }
    const int grid = (rows + 3) / 4;
    return launch(matvec_any_kernel<QT>, dim3(grid), dim3(256), 0, stream,
                  static_cast<const uint8_t*>(w), (int64_t)nb * F::kBytes, x, y, rows, nb);
}

static int matvec(const void* w, int qtype, const float* x, float* y, int rows, int cols,
                  hipStream_t stream) {
    int elems;
    switch (qtype) {
        case kQ4_0: elems = 32; break;
        case kQ8_0: elems = 32; break;
        case kQ4_K: elems = 256; break;
        case kQ6_K: elems = 256; break;
        default: return JINF_HIP_ERR_INVALID;
    }
    if (rows < 0 || cols < 0) return JINF_HIP_ERR_INVALID;
    if (rows == 0 || cols == 0) return JINF_HIP_OK;
    if (!w || !x || !y || cols % elems != 0) return JINF_HIP_ERR_INVALID;
    if (!aligned(x, 4) || !aligned(y, 4)) return JINF_HIP_ERR_INVALID;
    switch (qtype) {
        case kQ4_0: return matvec_t<kQ4_0>(w, x, y, rows, cols, stream);
        case kQ8_0: return matvec_t<kQ8_0>(w, x, y, rows, cols, stream);
        case kQ4_K: return matvec_t<kQ4_K>(w, x, y, rows, cols, stream);
        default: return matvec_t<kQ6_K>(w, x, y, rows, cols, stream);
    }
}

}  // namespace jinf

extern "C" int jinf_matvec_q4_0(const void* weight, const float* x, float* y, int rows,
                                int cols, hipStream_t stream) {
    return jinf::matvec(weight, jinf::kQ4_0, x, y, rows, cols, stream);
}

extern "C" int jinf_matvec(const void* weight, int qtype, const float* x, float* y, int rows,
                           int cols, hipStream_t stream) {
    return jinf::matvec(weight, qtype, x, y, rows, cols, stream);
}

// Drop-in for cuda/matmul_kernels.cu:198-225: Q4_0, Q8_0, Q4_K and Q6_K, as
// the reference; other qtypes are reported on stderr like its default branch.
extern "C" void jinf_cuda_dequant_matvec(const void* weight, const float* input, float* output,
                                         int rows, int cols, int qtype, hipStream_t stream) {
    if (rows == 0 || cols == 0) return;
    if (qtype != jinf::kQ4_0 && qtype != jinf::kQ8_0 && qtype != jinf::kQ4_K &&
        qtype != jinf::kQ6_K) {
        JINF_LOG("Unsupported qtype %d for dequant_matvec", qtype);
        return;
    }
    if (jinf::matvec(weight, qtype, input, output, rows, cols, stream) == JINF_HIP_ERR_INVALID)
        JINF_LOG("jinf_cuda_dequant_matvec: invalid argument (rows=%d cols=%d qtype=%d)", rows,
                 cols, qtype);
}
