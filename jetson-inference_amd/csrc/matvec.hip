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
//   - dequantisation is folded into the dot product: 4-bit codes (Q4_0,
//     Q4_K) meet x as exact integers, 8 products per v_dot8_i32_i4 against
//     x staged in fixed point as signed base-16 digit planes (plane_dot32);
//     8-bit and 6-bit codes (Q8_0, Q6_K) are multiplied as fp16 denormals
//     with v_fma_mix_f32 (see mix2); the per-block scale, offset and minimum
//     are applied once per block or sub-block;
//   - each row's lane partials meet in a DPP wave reduction.
// Anything the tiled kernel does not serve (unaligned pointers, widths that
// are not a multiple of the format's tile granule, more than 7 tiles) takes a
// one-wave-per-row kernel that decodes every weight exactly (quant_device.h).
#include <atomic>
#include <type_traits>

#include "jinf_device.h"
#include "jinf_host.h"
#include "quant_device.h"
#include "rope_device.h"
#include "jinf/kernels.h"
#include "jinf/kernels_ext.h"

namespace jinf {

constexpr int kMvTileElems = 4096;                // values of a row per column tile
constexpr int kMvLaneElems = kMvTileElems / kWave;  // 64 values per lane
constexpr int kMvMaxTiles = 7;                    // x of 7 tiles (112 KiB) fits in LDS
constexpr size_t kMvLdsBytes = 160 * 1024;        // LDS per workgroup on gfx950

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

// 2^-24 * sum_j q_j x_j for 8-bit codes q (0..255), four per word in value
// order: word i holds values 4i..4i+3 as bytes.
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

// ---- exact integer products for the 4-bit formats ----
//
// Q4_0 and Q4_K codes q (0..15) sit 8 to a dword (value 8i+n of a word group
// at bits 4n).  q ^ 8 read as a signed nibble is q - 8, so one
// v_dot8_i32_i4 gives sum_n (q_n - 8) D_n over 8 values for signed nibbles
// D_n: one VALU op for 8 weights, against 13 for the fp16-denormal products.
// For it each workgroup stages x once, per 32-value block:
//   X_j = rint(x_j 2^s) with s = 22 - e, e the exponent with max |x| < 2^e
//   (at least -100), so |X_j| <= 2^22;
//   X_j in six balanced base-16 digits, X_j = sum_p 16^p D_p, D_p in [-8, 7]:
//   the nibbles of (X_j + 0x888888) ^ 0x888888;
//   plane p of a word group: digit p of its 8 values, packed like the codes.
// Then sum_j (q_j - 8) X_j = sum_p 16^p P_p, P_p from six chains of dot8
// (exact: |P_p| <= 32 * 64), formed as lo + 4096 hi (both exact in fp32)
// with one rounding and scaled by 2^-s (exact).  Against fp32 x the only
// difference is X's rounding, at most 2^-23 of the block's largest |x| per
// value (the size of an fp32 product's own rounding for that value), and a
// one-hot x still gives d * (q - 8) exactly.  A block holding a non-finite
// x gives its rows NaN (the reference's fp32 products give NaN or +-inf).
constexpr int kMvRecWords = 52;  // a lane's planes: 48 digit words, 2 scales, 2 sums
constexpr int kMvRecTile16 = kMvRecWords * kWave / 4;  // 16-byte units per tile

// A lane's x for one tile, as its format consumes it.
struct MvXFloat {
    float v[kMvLaneElems];  // the lane's 64 values, prepared by the format
    float s[4];             // plain sums of values 16k .. 16k+15
};
struct MvXPlanes {
    uint32_t p[48];  // word group w (values 8w .. 8w+7 of the lane): digit k at 6w + k
    float inv[2];    // 2^-s of the lane's two 32-value blocks (NaN: non-finite x)
    int sx[2];       // sum of X over each block
};

// v_dot8_i32_i4 with a zero accumulator, in its three-operand form (the
// compiler picks the two-operand accumulate-in-place form and first moves a
// zero into the destination: six moves per block)
__device__ __forceinline__ int sdot8_first(int a, int b) {
    int r;
    asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// sum_j (q_j - 8) X_j + add over one 32-value block (code words q, planes
// pl[0..24)), rounded once to fp32.
__device__ __forceinline__ float plane_dot32(const uint32_t (&q)[4], const uint32_t* pl, int add) {
    int P[6];
    {
        const int qs = (int)(q[0] ^ 0x88888888u);
#pragma unroll
        for (int k = 0; k < 6; ++k) P[k] = sdot8_first(qs, (int)pl[k]);
    }
#pragma unroll
    for (int i = 1; i < 4; ++i) {
        const int qs = (int)(q[i] ^ 0x88888888u);
#pragma unroll
        for (int k = 0; k < 6; ++k)
            P[k] = __builtin_amdgcn_sdot8(qs, (int)pl[6 * i + k], P[k], false);
    }
    const int lo = (P[2] * 16 + P[1]) * 16 + P[0] + add;
    const int hi = (P[5] * 16 + P[4]) * 16 + P[3];
    return fmaf((float)hi, 4096.0f, (float)lo);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Stages word group g of the x tiles (values 8g .. 8g + 7: a, b) as planes.
// The four groups of a 32-value block are the four lanes of one quad and call
// this together.  Consumer lane l of tile t reads the record at
// rec + (64 t + l) * kMvRecWords: digit words [0, 48), 2^-s [48, 50), sums
// [50, 52).
__device__ __forceinline__ void mv_stage_planes(uint32_t* rec, int g, float4 a, float4 b) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    // block maximum of |x| as bit patterns (NaN and infinities compare above
    // every finite value)
    uint32_t mb = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) mb = max(mb, __float_as_uint(v[i]) & 0x7FFFFFFFu);
    mb = max(mb, dpp_u32<0xB1>(mb));  // quad_perm [1,0,3,2]
    mb = max(mb, dpp_u32<0x4E>(mb));  // quad_perm [2,3,0,1]
    const bool finite = mb < 0x7F800000u;
    const int e = max(__builtin_amdgcn_frexp_expf(__uint_as_float(mb)), -100);
    const float scale = ldexpf(1.0f, 22 - e);
    // X + 0x888888: x 2^s + 1.5 2^23 rounds x 2^s to an integer (|x 2^s| <=
    // 2^22), whose bits are 0x4B400000 + X.  (In a non-finite block these
    // are meaningless; the block's 2^-s is NaN.)
    uint32_t V[8];
    uint32_t us = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t u = __float_as_uint(fmaf(v[i], scale, 12582912.0f)) - (0x4B400000u - 0x888888u);
        us += u;
        V[i] = u ^ 0x888888u;
    }
    // digit pairs: byte c of t[k] = digits 2c of values 2k, 2k + 1 (low, high
    // nibble), byte c of u[k] = digits 2c + 1; then plane p = byte p / 2 of
    // t or u over k = 0..3
    uint32_t t[4], u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        t[k] = (V[2 * k] & 0x0F0F0F0Fu) | ((V[2 * k + 1] << 4) & 0xF0F0F0F0u);
        u[k] = ((V[2 * k] >> 4) & 0x0F0F0F0Fu) | (V[2 * k + 1] & 0xF0F0F0F0u);
    }
    uint32_t pl[6];
#pragma unroll
    for (int o = 0; o < 2; ++o) {
        const uint32_t* src = o ? u : t;
        const uint32_t a01 = __builtin_amdgcn_perm(src[1], src[0], 0x05010400u);
        const uint32_t a23 = __builtin_amdgcn_perm(src[3], src[2], 0x05010400u);
        const uint32_t b01 = __builtin_amdgcn_perm(src[1], src[0], 0x07030602u);
        const uint32_t b23 = __builtin_amdgcn_perm(src[3], src[2], 0x07030602u);
        pl[o] = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
        pl[2 + o] = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
        pl[4 + o] = __builtin_amdgcn_perm(b23, b01, 0x05040100u);
    }
    uint32_t* r = rec + (g >> 3) * kMvRecWords;  // consumer lane: 8 groups each
    uint2* d = reinterpret_cast<uint2*>(r + 6 * (g & 7));
    d[0] = make_uint2(pl[0], pl[1]);
    d[1] = make_uint2(pl[2], pl[3]);
    d[2] = make_uint2(pl[4], pl[5]);
    us += dpp_u32<0xB1>(us);
    us += dpp_u32<0x4E>(us);
    if ((g & 3) == 0) {
        const int blk = (g >> 2) & 1;
        r[48 + blk] = __float_as_uint(finite ? ldexpf(1.0f, e - 22) : __builtin_nanf(""));
        r[50 + blk] = us - 32u * 0x888888u;
    }
}

// ---- format policies for the tiled kernel ----
//
// Each gives the block geometry, the width granule of the fast path (a
// multiple that makes row and tile byte counts multiples of 16), the rows per
// item, the lane's x representation (kPlanes: MvXPlanes, else MvXFloat with
// its values prepared by prep) and the lane's dot product over its 64 values
// of one staged row tile (`row`: the tile's bytes in LDS as dwords).

template <int QT> struct MvFmt;

// Q4_0: lane = 2 consecutive blocks (36 B, 9 dwords at 9 * lane: conflict
// free).  y += (d 2^-s) sum (q - 8) X per block (plane_dot32).
template <> struct MvFmt<kQ4_0> {
    static constexpr int kElems = 32, kBytes = 18, kColGranule = 256, kRows = 2;
    static constexpr bool kPlanes = true;
    using XReg = MvXPlanes;
    static __device__ float dot(const uint32_t* row, int lane, const XReg& x) {
        const uint32_t* l = row + 9 * lane;
        uint32_t D[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) D[i] = l[i];
        const float d0 = h2f((uint16_t)(D[0] & 0xFFFFu));
        const float d1 = h2f((uint16_t)(D[4] >> 16));
        const uint32_t q0[4] = {__builtin_amdgcn_alignbit(D[1], D[0], 16),
                                __builtin_amdgcn_alignbit(D[2], D[1], 16),
                                __builtin_amdgcn_alignbit(D[3], D[2], 16),
                                __builtin_amdgcn_alignbit(D[4], D[3], 16)};
        const uint32_t q1[4] = {D[5], D[6], D[7], D[8]};
        const float t0 = plane_dot32(q0, x.p, 0);
        const float t1 = plane_dot32(q1, x.p + 24, 0);
        return fmaf(d1 * x.inv[1], t1, (d0 * x.inv[0]) * t0);
    }
};

// Q8_0: lane = 2 consecutive blocks (68 B, 17 dwords at 17 * lane: conflict
// free).  The int8 codes are biased to unsigned (q ^ 0x80 = q + 128) for the
// fp16-denormal product, and the bias comes back as -128 * sum x per block.
template <> struct MvFmt<kQ8_0> {
    static constexpr int kElems = 32, kBytes = 34, kColGranule = 256, kRows = 1;
    static constexpr bool kPlanes = false;
    using XReg = MvXFloat;
    static __device__ void prep(float (&)[64]) {}
    static __device__ float dot(const uint32_t* row, int lane, const XReg& x) {
        const float (&xv)[64] = x.v;
        const float (&xs)[4] = x.s;
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
// lanes) and 8 dwords of nibbles.  Per sub-block (one 32-value x block):
//   sum_j (sub_d q_j - sub_min) x_j
//     = 2^-s (sub_d sum q X - sub_min sum X),  sum q X = sum (q - 8) X + 8 sum X.
template <> struct MvFmt<kQ4_K> {
    static constexpr int kElems = 256, kBytes = 144, kColGranule = 256, kRows = 2;
    static constexpr bool kPlanes = true;
    using XReg = MvXPlanes;
    static __device__ float dot(const uint32_t* row, int lane, const XReg& x) {
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
        const float d = h2f((uint16_t)(h & 0xFFFFu));
        const float dmin = h2f((uint16_t)(h >> 16));
        int sc0, mn0, sc1, mn1;
        q4_K_scale_min(s, 2 * k, sc0, mn0);
        q4_K_scale_min(s, 2 * k + 1, sc1, mn1);
        const float u0 = plane_dot32(q0, x.p, 8 * x.sx[0]);
        const float u1 = plane_dot32(q1, x.p + 24, 8 * x.sx[1]);
        const float t0 = fmaf(d * (float)sc0, u0, -(dmin * (float)mn0) * (float)x.sx[0]) * x.inv[0];
        const float t1 = fmaf(d * (float)sc1, u1, -(dmin * (float)mn1) * (float)x.sx[1]) * x.inv[1];
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
    static constexpr bool kPlanes = false;
    using XReg = MvXFloat;
    static __device__ void prep(float (&)[64]) {}
    static __device__ float dot(const uint32_t* row, int lane, const XReg& x) {
        const float (&xv)[64] = x.v;
        const float (&xs)[4] = x.s;
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

template <int QT, int R> struct MvTile {
    using F = MvFmt<QT>;
    static constexpr int kTileBlocks = kMvTileElems / F::kElems;
    static constexpr int kTileBytes = kTileBlocks * F::kBytes;
    static constexpr int kChunks = kTileBytes / 16;
    static constexpr int kCPL = (kChunks + kWave - 1) / kWave;  // 16-byte chunks per lane
    // chunk slots past a row's kChunks that the last pass writes (see stage)
    static constexpr int kPad = kWave * kCPL - kChunks;
    static constexpr int kStageChunks = R * kChunks + kPad;  // per wave
    static_assert(kTileBytes % 16 == 0, "tile must be whole 16-byte chunks");
    static_assert(kPad < kWave, "pad must be rewritten by the first pass");
};

// x tile layout in LDS: tile t holds 1024 float4 (4096 floats); lane l's 16
// float4 sit in row l with the column XOR-swizzled by l & 15, so the 16 lanes
// of one LDS pass read 16 distinct bank groups.
__device__ __forceinline__ int mv_xslot(int tile, int l, int j) {
    return (tile << 10) + (l << 4) + (j ^ (l & 15));
}

// ---- what a launch computes around the dot products ----
//
// Prologue (the x the rows are multiplied with):
//   kProNone  x as given;
//   kProNorm  x_j = fl32(fl32(h_j * rs) * g_j), rs from the fp64 sum of h_j^2
//             (rms_scale): the reference's RMSNorm launch feeding the GEMV
//             (cuda/rmsnorm_kernel.cu:9-61), computed by every workgroup.
// Epilogue (what happens to a finished row value v):
//   kEpiStore  y[row] = v;
//   kEpiAdd    y[row] = y[row] + v: the residual add after the output and
//              down projections (src/engine.cpp:466, :508);
//   kEpiSwiGLU a group is row r of W_gate and row r of W_up:
//              y[r] = swiglu_exact(v_gate, v_up) (src/engine.cpp:489-502);
//   kEpiQKV    rows of up to three matrices (q, k, v segments), a group is two
//              consecutive rows = one RoPE pair: q pairs are rotated and
//              stored to y, k pairs rotated and stored into the K cache row
//              at *pos, v pairs stored into the V cache row
//              (src/engine.cpp:432-453).
enum MvPro { kProNone = 0, kProNorm = 1 };
enum MvEpi { kEpiStore = 0, kEpiAdd = 1, kEpiSwiGLU = 2, kEpiQKV = 3 };

// The fields the first loads (x, the norm weight, the first weight rows)
// need come first: the first 14 dwords of the kernel arguments arrive
// preloaded in SGPRs.
struct MvJob {
    const float* x;         // x, or h for kProNorm
    const void* norm_w;     // kProNorm: g (fp32 or fp16)
    const uint8_t* W[3];    // segment matrices (same format and width)
    int64_t row_bytes;
    int rows;               // virtual rows; kEpiSwiGLU: output rows
    int nb;                 // blocks per row
    int nt;                 // column tiles
    int seg_end[3];         // kEpiQKV: virtual row where each segment ends
    int norm_f16;
    float eps;
    float* y;
    void* kc;               // kEpiQKV: K / V cache rows [max_ctx][kv_dim]
    void* vc;
    const int32_t* pos;
    int kv_f16, kv_dim, head_dim, max_ctx;
};

struct NoTheta {};
template <int EPI> using MvTheta = typename std::conditional<EPI == kEpiQKV, RopeTheta, NoTheta>::type;

// Rows per work item: a row pair for the pair epilogues; otherwise the
// format's own count, raised to 2 when each group walks several tiles (WIDE):
// there more rows per item shorten each wave's chain of items (Q6_K down
// projection 4096 x 14336: 17.1 us against 20.1 with one row), while on
// single-tile matrices one row keeps more items in flight (Q6_K 4096 x 4096:
// 6.2 us against 7.0).
template <int QT, int EPI, bool WIDE = false> struct MvGroup {
    static constexpr bool kPairs = EPI == kEpiSwiGLU || EPI == kEpiQKV;
    static constexpr int kFmtRows = MvFmt<QT>::kRows;
    static constexpr int R = kPairs ? 2 : (WIDE && kFmtRows < 2 ? 2 : kFmtRows);
    static __device__ __host__ int groups(const MvJob& j) {
        return EPI == kEpiSwiGLU ? j.rows : (j.rows + R - 1) / R;
    }
};

// Row r of group g (clamped into the matrix: groups past the end re-read the
// last row, whose result is never stored).
template <int QT, int EPI, bool WIDE = false>
__device__ __forceinline__ const uint8_t* mv_row(const MvJob& j, int g, int r) {
    constexpr int R = MvGroup<QT, EPI, WIDE>::R;
    if constexpr (EPI == kEpiSwiGLU) {
        const int row = g < j.rows ? g : j.rows - 1;
        return j.W[r] + (int64_t)row * j.row_bytes;
    } else {
        int v = g * R + r;
        if (v >= j.rows) v = j.rows - 1;
        if constexpr (EPI == kEpiQKV) {
            const int s = v < j.seg_end[0] ? 0 : v < j.seg_end[1] ? 1 : 2;
            const int start = s == 0 ? 0 : j.seg_end[s - 1];
            return j.W[s] + (int64_t)(v - start) * j.row_bytes;
        } else {
            return j.W[0] + (int64_t)v * j.row_bytes;
        }
    }
}

template <typename T>
__device__ __forceinline__ void cache_store(void* c, int64_t i, float a, float b) {
    T* p = static_cast<T*>(c) + i;
    if constexpr (sizeof(T) == 2) {
        p[0] = f2h(a);
        p[1] = f2h(b);
    } else {
        p[0] = a;
        p[1] = b;
    }
}

// Finished values v[0..R) of group g (one lane).  yo: kEpiAdd's y values of
// the group's rows, loaded ahead (NULL: read here); pos: kEpiQKV's position;
// rcs: its (cos, sin) table for the position (NULL: computed here).
template <int QT, int EPI, bool WIDE = false>
__device__ __forceinline__ void mv_epilogue(const MvJob& j, const MvTheta<EPI>& th, int g,
                                            float (&v)[MvGroup<QT, EPI, WIDE>::R],
                                            const float* yo, int pos,
                                            const float2* rcs = nullptr) {
    constexpr int R = MvGroup<QT, EPI, WIDE>::R;
    if constexpr (EPI == kEpiStore) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (g * R + r < j.rows) j.y[g * R + r] = v[r];
    } else if constexpr (EPI == kEpiAdd) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (g * R + r < j.rows) j.y[g * R + r] = (yo ? yo[r] : j.y[g * R + r]) + v[r];
    } else if constexpr (EPI == kEpiSwiGLU) {
        if (g < j.rows) j.y[g] = swiglu_exact(v[0], v[1]);
    } else {
        const int v0 = 2 * g;
        if (v0 >= j.rows) return;
        const int s = v0 < j.seg_end[0] ? 0 : v0 < j.seg_end[1] ? 1 : 2;
        const int local = v0 - (s == 0 ? 0 : j.seg_end[s - 1]);
        float a = v[0], b = v[1];
        if (s < 2) {
            const int i = (local % j.head_dim) / 2;
            const float2 cs = rcs ? rcs[i] : rope_cs(pos, th.t[i]);
            rot(a, b, cs.x, cs.y);
        }
        if (s == 0) {
            j.y[local] = a;
            j.y[local + 1] = b;
        } else if (pos >= 0 && pos < j.max_ctx) {
            void* c = s == 1 ? j.kc : j.vc;
            const int64_t i = (int64_t)pos * j.kv_dim + local;
            if (j.kv_f16)
                cache_store<uint16_t>(c, i, a, b);
            else
                cache_store<float>(c, i, a, b);
        }
    }
}

// Whether the kernel defers its epilogue to the end (at most 64 groups per
// wave).  (Deferring the q / k / v epilogue as well measured 6.5 against 6.3
// us: its groups are few per wave.)
constexpr bool mv_defers(int epi) { return epi == kEpiSwiGLU; }

// Each wave takes whole groups of R rows (groups g, g + stride, ...) and
// walks their tiles in order, so a row's partial sums stay in registers until
// its last tile.  The wave's LDS accesses execute in order; the fences keep
// the compiler from moving the read-back above the stores.  Workgroup
// barriers only follow the x staging.
// WV1: waves of a one-tile workgroup (4, or 8 where the kernel fits four
// waves per SIMD: one x staging for twice the waves).  TALL: a one-tile
// matrix with the wide row grouping (two rows per item for the one-row
// formats), for very tall matrices.  XW: float4 of x each thread of a wide
// workgroup loads (enough for its tiles; loads past them are branches).
template <int QT, bool ONE_TILE, int PRO, int EPI, int WV1, bool TALL = false, int XW = 28>
__global__ __launch_bounds__(ONE_TILE ? 64 * WV1 : 512) void matvec_kernel(MvJob job,
                                                                           MvTheta<EPI> th) {
#define MV_BID blockIdx.x
#define MV_NBLK gridDim.x
#include "matvec_body.inc"
#undef MV_BID
#undef MV_NBLK
}

// Any width / alignment: one wave per group of R rows; each lane takes
// 8-value groups with stride 64, decodes them exactly (byte loads) and fmas
// them with x (with kProNorm, x_j is formed on the fly from h_j and g_j).
template <int QT, int PRO, int EPI>
__global__ __launch_bounds__(256) void matvec_any_kernel(MvJob job, MvTheta<EPI> th) {
    constexpr int E = QGeom<QT>::kElems, B = QGeom<QT>::kBytes;
    constexpr int R = MvGroup<QT, EPI>::R;
    const int lane = threadIdx.x & (kWave - 1);
    const int g = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (g >= MvGroup<QT, EPI>::groups(job)) return;
    const int n8 = job.nb * (E / 8);
    float rs = 1.0f;
    if constexpr (PRO == kProNorm) {
        double ss = 0.0;
        for (int j = lane; j < 8 * n8; j += kWave) ss = fma((double)job.x[j], (double)job.x[j], ss);
        rs = rms_scale(wave_sum(ss), 8 * n8, job.eps);
    }
    const uint8_t* wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r] = mv_row<QT, EPI>(job, g, r);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (int gi = lane; gi < n8; gi += kWave) {
        const int b = gi / (E / 8);
        const int e0 = (gi % (E / 8)) * 8;
        float xv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int j = 8 * gi + i;
            float xj = job.x[j];
            if constexpr (PRO == kProNorm) {
#pragma clang fp contract(off)
                const float w = job.norm_f16 ? h2f(static_cast<const uint16_t*>(job.norm_w)[j])
                                             : static_cast<const float*>(job.norm_w)[j];
                xj = (xj * rs) * w;
            }
            xv[i] = xj;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float w[8];
            decode8<QT>(wr[r] + (int64_t)b * B, e0, w);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[r] = fmaf(w[i], xv[i], acc[r]);
        }
    }
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = wave_sum_f32(acc[r]);
    if (lane == 0) mv_epilogue<QT, EPI>(job, th, g, v, nullptr, EPI == kEpiQKV ? job.pos[0] : 0);
}

// Host checks shared with the two-format Q/K/V launch (matvec_qkv2.hip).
static int q_elems(int qtype) {
    switch (qtype) {
        case kQ4_0: case kQ8_0: return 32;
        case kQ4_K: case kQ6_K: return 256;
        default: return 0;
    }
}

// Common checks: a served qtype, whole blocks, 4-byte aligned vectors.
static int mv_check(int qtype, int rows, int cols, const float* x, const float* y) {
    const int e = q_elems(qtype);
    if (e == 0 || rows < 0 || cols < 0) return JINF_HIP_ERR_INVALID;
    if (rows == 0 || cols == 0) return -1;  // nothing to do
    if (!x || !y || cols % e != 0) return JINF_HIP_ERR_INVALID;
    if (!aligned(x, 4) || !aligned(y, 4)) return JINF_HIP_ERR_INVALID;
    return JINF_HIP_OK;
}

static int norm_setup(MvJob& j, const void* norm_w, int norm_type, float eps) {
    j.norm_w = norm_w;
    j.norm_f16 = norm_type == JINF_HIP_F16;
    j.eps = eps;
    if (!norm_w) return JINF_HIP_OK;
    if (norm_type != JINF_HIP_F32 && norm_type != JINF_HIP_F16) return JINF_HIP_ERR_INVALID;
    if (!aligned(norm_w, norm_type == JINF_HIP_F16 ? 2 : 4) || !(eps >= 0.0f))
        return JINF_HIP_ERR_INVALID;
    return JINF_HIP_OK;
}

// The Q/K/V job of jinf_rmsnorm_qkv_rope after its checks; *none when there
// is nothing to compute.
static int qkv_job(MvJob& j, bool* none, const void* wq, const void* wk, const void* wv,
                   int qtype, const float* h, const void* norm_w, int norm_type, float eps,
                   int cols, float* q_out, void* k_cache, void* v_cache, int kv_type,
                   const int32_t* pos, int max_ctx, int head_dim, int n_heads, int n_heads_kv,
                   float freq_base) {
    *none = true;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim / 2 > kRopeMaxHalf || n_heads < 0 ||
        n_heads_kv < 0 || max_ctx < 0)
        return JINF_HIP_ERR_INVALID;
    if (kv_type != JINF_HIP_F32 && kv_type != JINF_HIP_F16) return JINF_HIP_ERR_INVALID;
    if (!(freq_base > 0.0f)) return JINF_HIP_ERR_INVALID;
    const int64_t qd = (int64_t)n_heads * head_dim, kvd = (int64_t)n_heads_kv * head_dim;
    const int64_t rq = wq ? qd : 0, rk = wk ? kvd : 0, rv = wv ? kvd : 0;
    if (rq + rk + rv > 0x7FFFFFFF) return JINF_HIP_ERR_INVALID;
    const int rows = (int)(rq + rk + rv);
    if (rows == 0) return JINF_HIP_OK;
    if ((wq && !q_out) || (wk && !k_cache) || (wv && !v_cache) || !pos)
        return JINF_HIP_ERR_INVALID;
    if (q_out && !aligned(q_out, 4)) return JINF_HIP_ERR_INVALID;
    const int es = kv_type == JINF_HIP_F16 ? 2 : 4;
    if ((k_cache && !aligned(k_cache, es)) || (v_cache && !aligned(v_cache, es)))
        return JINF_HIP_ERR_INVALID;
    const int c = mv_check(qtype, rows, cols, h, q_out ? q_out : h);
    if (c != JINF_HIP_OK) return c < 0 ? JINF_HIP_OK : c;
    j = MvJob{};
    if (norm_setup(j, norm_w, norm_type, eps) != JINF_HIP_OK) return JINF_HIP_ERR_INVALID;
    // q, k, v segments in that order; an absent one is empty
    const void* first = wq ? wq : wk ? wk : wv;
    j.W[0] = static_cast<const uint8_t*>(wq ? wq : first);
    j.W[1] = static_cast<const uint8_t*>(wk ? wk : first);
    j.W[2] = static_cast<const uint8_t*>(wv ? wv : first);
    j.seg_end[0] = (int)rq;
    j.seg_end[1] = (int)(rq + rk);
    j.seg_end[2] = rows;
    j.rows = rows;
    j.x = h;
    j.y = q_out;
    j.kc = k_cache;
    j.vc = v_cache;
    j.pos = pos;
    j.kv_f16 = kv_type == JINF_HIP_F16;
    j.kv_dim = (int)kvd;
    j.head_dim = head_dim;
    j.max_ctx = max_ctx;
    *none = false;
    return JINF_HIP_OK;
}

#ifndef JINF_MATVEC_KERNELS_ONLY

// Workgroups of the tall one-tile kernel (these template arguments, `threads`
// lanes, `shmem` bytes) that the device holds at once: its occupancy per CU
// times the CUs.  Such a launch streams tens of items per wave, so it takes
// every resident slot (the RMSNorm + Q6_K output head, 128256 x 4096, three
// workgroups per CU: 80.0 -> 76.0-76.9 us at 768 workgroups against 512).
// Queried once per kernel and process, on the current device (metadata
// queries only, so also under stream capture; a process whose devices differ
// uses the first one's figure); 512 if a query fails.  The grid changes no
// row's arithmetic, so no result depends on it.
template <int QT, int PRO, int EPI, int WV1>
static int mv_tall_grid_cap(int threads, size_t shmem) {
    static std::atomic<int> cap{0};
    int c = cap.load(std::memory_order_relaxed);
    if (c > 0) return c;
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, matvec_kernel<QT, true, PRO, EPI, WV1, true>, threads, shmem) != hipSuccess ||
        per_cu < 1 || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
        return 512;
    c = per_cu * cus;
    cap.store(c, std::memory_order_relaxed);
    return c;
}

// Launch a job: the tiled kernel with at most 512 workgroups when the shape
// and alignment allow it (single-tile matrices use 4 independent waves per
// workgroup; wider ones 8 waves sharing one copy of x), else the
// one-wave-per-group kernel.
template <int QT, int PRO, int EPI>
static int mv_run(MvJob job, int cols, const MvTheta<EPI>& th, hipStream_t stream) {
    using F = MvFmt<QT>;
    // 8-wave one-tile workgroups where the kernel fits four waves per SIMD:
    // Q4_0, except the fused q / k / v launch (154 VGPRs; with its epilogue
    // deferred it fits, but its 1.5 groups per wave then ran 7.9 against 6.5 us)
    constexpr int WV1 = QT == kQ4_0 && EPI != kEpiQKV ? 8 : 4;
    using G = MvGroup<QT, EPI>;
    using GW = MvGroup<QT, EPI, true>;
    job.nb = cols / F::kElems;
    job.row_bytes = (int64_t)job.nb * F::kBytes;
    job.nt = (cols + kMvTileElems - 1) / kMvTileElems;
    // Very tall one-tile matrices of the one-row formats (the output head,
    // 128256 x 4096 Q6_K: 100 against 106 us) take two rows per item.
    constexpr bool kTallable = F::kRows == 1 && EPI == kEpiStore;
    const bool tall = kTallable && job.nt == 1 && job.rows >= 32768;
    const int n_groups = job.nt == 1 && !tall ? G::groups(job) : GW::groups(job);
    bool tiled = cols % F::kColGranule == 0 && job.nt <= kMvMaxTiles && aligned(job.x, 16);
    for (int s = 0; s < 3; ++s) tiled = tiled && aligned(job.W[s], 16);
    if (PRO == kProNorm) tiled = tiled && aligned(job.norm_w, job.norm_f16 ? 8 : 16);
    if (tiled) {
        const int stage_chunks = job.nt == 1 && !tall ? MvTile<QT, G::R>::kStageChunks
                                                      : MvTile<QT, GW::R>::kStageChunks;
        // one-tile matrices: WV1 waves; wide ones: 8 waves share one copy of
        // x, 4 where 8 staging regions and x would not fit in the 160 KiB of
        // LDS (7-tile Q8_0 / Q6_K)
        constexpr int xt16 = F::kPlanes ? kMvRecTile16 : 1024;  // x per tile, 16-byte units
        int waves = job.nt == 1 ? WV1 : 8;
        if ((size_t)(job.nt * xt16 + waves * stage_chunks) * 16 > kMvLdsBytes) waves = 4;
        int grid = (n_groups + waves - 1) / waves;
        // 512 workgroups (two per CU on 256 CUs) measured best for Q4_0 at
        // 4096-14336 rows; each wave then streams several items.  Deferred
        // epilogues hold one finished group per lane: at most 64 per wave.
        if (grid > 512) grid = 512;
        if (mv_defers(EPI) && (int64_t)grid * waves * kWave < n_groups)
            grid = (int)(((int64_t)n_groups + waves * kWave - 1) / (waves * kWave));
        const size_t shmem = ((size_t)job.nt * xt16 + (size_t)waves * stage_chunks) * 16;
        if constexpr (kTallable) {
            if (tall) {
                const int cap = mv_tall_grid_cap<QT, PRO, EPI, WV1>(waves * kWave, shmem);
                const int want = (n_groups + waves - 1) / waves;
                return launch(matvec_kernel<QT, true, PRO, EPI, WV1, true>,
                              dim3(want < cap ? want : cap), dim3(waves * kWave), shmem, stream,
                              job, th);
            }
        }
        if (job.nt == 1)
            return launch(matvec_kernel<QT, true, PRO, EPI, WV1>, dim3(grid), dim3(waves * kWave),
                          shmem, stream, job, th);
        // x float4 per thread for the wide kernel: nt tiles of 1024 float4
        const int xw = (job.nt * 1024 + waves * kWave - 1) / (waves * kWave);
        if (xw <= 4)
            return launch(matvec_kernel<QT, false, PRO, EPI, 4, false, 4>, dim3(grid),
                          dim3(waves * kWave), shmem, stream, job, th);
        if (xw <= 8)
            return launch(matvec_kernel<QT, false, PRO, EPI, 4, false, 8>, dim3(grid),
                          dim3(waves * kWave), shmem, stream, job, th);
        if (xw <= 14)
            return launch(matvec_kernel<QT, false, PRO, EPI, 4, false, 14>, dim3(grid),
                          dim3(waves * kWave), shmem, stream, job, th);
        return launch(matvec_kernel<QT, false, PRO, EPI, 4, false, 28>, dim3(grid),
                      dim3(waves * kWave), shmem, stream, job, th);
    }
    const int any_groups = G::groups(job);
    if ((any_groups + 3) / 4 > 0x7FFFFFFF / 4) return JINF_HIP_ERR_INVALID;
    return launch(matvec_any_kernel<QT, PRO, EPI>, dim3((any_groups + 3) / 4), dim3(256), 0,
                  stream, job, th);
}

template <int PRO, int EPI>
static int mv_dispatch(int qtype, const MvJob& job, int cols, const MvTheta<EPI>& th,
                       hipStream_t stream) {
    switch (qtype) {
        case kQ4_0: return mv_run<kQ4_0, PRO, EPI>(job, cols, th, stream);
        case kQ8_0: return mv_run<kQ8_0, PRO, EPI>(job, cols, th, stream);
        case kQ4_K: return mv_run<kQ4_K, PRO, EPI>(job, cols, th, stream);
        case kQ6_K: return mv_run<kQ6_K, PRO, EPI>(job, cols, th, stream);
        default: return JINF_HIP_ERR_INVALID;
    }
}

static int matvec(const void* w, int qtype, const float* x, float* y, int rows, int cols,
                  hipStream_t stream) {
    const int c = mv_check(qtype, rows, cols, x, y);
    if (c != JINF_HIP_OK) return c < 0 ? JINF_HIP_OK : c;
    if (!w) return JINF_HIP_ERR_INVALID;
    MvJob j{};
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(w);
    j.rows = rows;
    j.x = x;
    j.y = y;
    return mv_dispatch<kProNone, kEpiStore>(qtype, j, cols, NoTheta{}, stream);
}

static int rmsnorm_matvec(const void* w, int qtype, const float* h, const void* norm_w,
                          int norm_type, float eps, float* y, int rows, int cols,
                          hipStream_t stream) {
    const int c = mv_check(qtype, rows, cols, h, y);
    if (c != JINF_HIP_OK) return c < 0 ? JINF_HIP_OK : c;
    if (!w) return JINF_HIP_ERR_INVALID;
    MvJob j{};
    if (norm_setup(j, norm_w, norm_type, eps) != JINF_HIP_OK) return JINF_HIP_ERR_INVALID;
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(w);
    j.rows = rows;
    j.x = h;
    j.y = y;
    if (!norm_w) return mv_dispatch<kProNone, kEpiStore>(qtype, j, cols, NoTheta{}, stream);
    return mv_dispatch<kProNorm, kEpiStore>(qtype, j, cols, NoTheta{}, stream);
}

static int matvec_add(const void* w, int qtype, const float* x, float* y, int rows, int cols,
                      hipStream_t stream) {
    const int c = mv_check(qtype, rows, cols, x, y);
    if (c != JINF_HIP_OK) return c < 0 ? JINF_HIP_OK : c;
    if (!w) return JINF_HIP_ERR_INVALID;
    MvJob j{};
    j.W[0] = j.W[1] = j.W[2] = static_cast<const uint8_t*>(w);
    j.rows = rows;
    j.x = x;
    j.y = y;
    return mv_dispatch<kProNone, kEpiAdd>(qtype, j, cols, NoTheta{}, stream);
}

static int rmsnorm_swiglu_matvec(const void* wg, const void* wu, int qtype, const float* h,
                                 const void* norm_w, int norm_type, float eps, float* out,
                                 int n_ff, int cols, hipStream_t stream) {
    const int c = mv_check(qtype, n_ff, cols, h, out);
    if (c != JINF_HIP_OK) return c < 0 ? JINF_HIP_OK : c;
    if (!wg || !wu) return JINF_HIP_ERR_INVALID;
    MvJob j{};
    if (norm_setup(j, norm_w, norm_type, eps) != JINF_HIP_OK) return JINF_HIP_ERR_INVALID;
    j.W[0] = static_cast<const uint8_t*>(wg);
    j.W[1] = static_cast<const uint8_t*>(wu);
    j.W[2] = j.W[0];
    j.rows = n_ff;
    j.x = h;
    j.y = out;
    if (!norm_w) return mv_dispatch<kProNone, kEpiSwiGLU>(qtype, j, cols, NoTheta{}, stream);
    return mv_dispatch<kProNorm, kEpiSwiGLU>(qtype, j, cols, NoTheta{}, stream);
}

static int rmsnorm_qkv_rope(const void* wq, const void* wk, const void* wv, int qtype,
                            const float* h, const void* norm_w, int norm_type, float eps,
                            int cols, float* q_out, void* k_cache, void* v_cache, int kv_type,
                            const int32_t* pos, int max_ctx, int head_dim, int n_heads,
                            int n_heads_kv, float freq_base, hipStream_t stream) {
    MvJob j;
    bool none;
    const int rc = qkv_job(j, &none, wq, wk, wv, qtype, h, norm_w, norm_type, eps, cols, q_out,
                           k_cache, v_cache, kv_type, pos, max_ctx, head_dim, n_heads,
                           n_heads_kv, freq_base);
    if (rc != JINF_HIP_OK || none) return rc;
    RopeTheta th;
    theta_table(th, head_dim, freq_base);
    if (!norm_w) return mv_dispatch<kProNone, kEpiQKV>(qtype, j, cols, th, stream);
    return mv_dispatch<kProNorm, kEpiQKV>(qtype, j, cols, th, stream);
}

#endif  // JINF_MATVEC_KERNELS_ONLY

}  // namespace jinf

#ifndef JINF_MATVEC_KERNELS_ONLY

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

extern "C" int jinf_rmsnorm_matvec(const void* weight, int qtype, const float* h,
                                   const void* norm_w, int norm_type, float eps, float* y,
                                   int rows, int cols, hipStream_t stream) {
    return jinf::rmsnorm_matvec(weight, qtype, h, norm_w, norm_type, eps, y, rows, cols, stream);
}

extern "C" int jinf_matvec_add(const void* weight, int qtype, const float* x, float* y, int rows,
                               int cols, hipStream_t stream) {
    return jinf::matvec_add(weight, qtype, x, y, rows, cols, stream);
}

extern "C" int jinf_rmsnorm_swiglu_matvec(const void* w_gate, const void* w_up, int qtype,
                                          const float* h, const void* norm_w, int norm_type,
                                          float eps, float* out, int n_ff, int cols,
                                          hipStream_t stream) {
    return jinf::rmsnorm_swiglu_matvec(w_gate, w_up, qtype, h, norm_w, norm_type, eps, out, n_ff,
                                       cols, stream);
}

extern "C" int jinf_rmsnorm_qkv_rope(const void* w_q, const void* w_k, const void* w_v, int qtype,
                                     const float* h, const void* norm_w, int norm_type, float eps,
                                     int cols, float* q_out, void* k_cache, void* v_cache,
                                     int kv_type, const int32_t* pos, int max_ctx, int head_dim,
                                     int n_heads, int n_heads_kv, float freq_base,
                                     hipStream_t stream) {
    return jinf::rmsnorm_qkv_rope(w_q, w_k, w_v, qtype, h, norm_w, norm_type, eps, cols, q_out,
                                  k_cache, v_cache, kv_type, pos, max_ctx, head_dim, n_heads,
                                  n_heads_kv, freq_base, stream);
}

#endif  // JINF_MATVEC_KERNELS_ONLY
