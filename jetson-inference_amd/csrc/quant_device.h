// GGUF weight block formats served on the GPU (reference
// include/jinf/quant.h:8-68): geometry and an exact per-element decode.
//
//   Q4_0  (qtype 2)  18 B / 32 values:  d (binary16), qs[16]
//   Q8_0  (qtype 8)  34 B / 32 values:  d (binary16), int8 qs[32]
//   Q4_K  (qtype 12) 144 B / 256 values: d, dmin (binary16), scales[12], qs[128]
//   Q6_K  (qtype 14) 210 B / 256 values: ql[128], qh[64], int8 scales[16], d
//
// decode8 reproduces the reference's dequantized fp32 weights bit for bit
// (src/quant.cpp:49-105, cuda/dequant_kernels.cu:6-110): Q4_0, Q8_0 and Q6_K
// weights are exact products; a Q4_K weight is sub_d * q - sub_min with an
// exact product, so its single rounding is the same with or without FMA
// contraction.  Blocks are read with byte loads, so any alignment works.
#pragma once

#include "jinf_device.h"

namespace jinf {

constexpr int kQ4_0 = 2;
constexpr int kQ8_0 = 8;
constexpr int kQ4_K = 12;
constexpr int kQ6_K = 14;

template <int QT> struct QGeom;
template <> struct QGeom<kQ4_0> { static constexpr int kElems = 32, kBytes = 18; };
template <> struct QGeom<kQ8_0> { static constexpr int kElems = 32, kBytes = 34; };
template <> struct QGeom<kQ4_K> { static constexpr int kElems = 256, kBytes = 144; };
template <> struct QGeom<kQ6_K> { static constexpr int kElems = 256, kBytes = 210; };

__device__ __forceinline__ float ld_f16_bytes(const uint8_t* p) {
    return h2f((uint16_t)(p[0] | (p[1] << 8)));
}

// The reference's unpacking of the Q4_K 12-byte scale array for sub-block sb
// (src/quant.cpp:70-75): sub-blocks 0-3 use the low six bits of bytes sb
// (scale) and sb + 4 (min); sub-blocks 4-7 take a nibble of byte sb + 4 as
// their high four bits and the top two bits of byte sb - 4 (scale) or sb
// (min) as their low two.  Byte k of the array is (s[k / 4] >> 8 (k % 4)).
__device__ __forceinline__ void q4_K_scale_min(const uint32_t (&s)[3], int sb, int& sc, int& mn) {
    auto byte = [&](int k) -> int { return (int)((s[k >> 2] >> (8 * (k & 3))) & 0xFFu); };
    if (sb < 4) {
        sc = byte(sb) & 0x3F;
        mn = byte(sb + 4) & 0x3F;
    } else {
        const int i = sb - 4;
        sc = ((byte(i + 8) & 0x0F) << 2) | (byte(i) >> 6);
        mn = ((byte(i + 8) >> 4) << 2) | (byte(i + 4) >> 6);
    }
}

// Weights e0 .. e0+7 (e0 % 8 == 0) of one block starting at blk.
template <int QT>
__device__ __forceinline__ void decode8(const uint8_t* blk, int e0, float (&w)[8]) {
    if constexpr (QT == kQ4_0) {
        const float d = ld_f16_bytes(blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t b = blk[2 + e0 / 2 + i];
            w[2 * i] = (float)((int)(b & 0x0F) - 8) * d;
            w[2 * i + 1] = (float)((int)(b >> 4) - 8) * d;
        }
    } else if constexpr (QT == kQ8_0) {
        const float d = ld_f16_bytes(blk);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (float)(int8_t)blk[2 + e0 + i] * d;
    } else if constexpr (QT == kQ4_K) {
        const float d = ld_f16_bytes(blk);
        const float dmin = ld_f16_bytes(blk + 2);
        uint32_t s[3];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            s[k] = (uint32_t)blk[4 + 4 * k] | ((uint32_t)blk[5 + 4 * k] << 8) |
                   ((uint32_t)blk[6 + 4 * k] << 16) | ((uint32_t)blk[7 + 4 * k] << 24);
        int sc, mn;
        q4_K_scale_min(s, e0 / 32, sc, mn);
        const float sub_d = d * (float)sc;
        const float sub_min = dmin * (float)mn;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t b = blk[16 + e0 / 2 + i];
            w[2 * i] = __builtin_fmaf(sub_d, (float)(b & 0x0F), -sub_min);
            w[2 * i + 1] = __builtin_fmaf(sub_d, (float)(b >> 4), -sub_min);
        }
    } else {
        static_assert(QT == kQ6_K, "unsupported block type");
        const float scale = ld_f16_bytes(blk + 208) * (float)(int8_t)blk[192 + e0 / 16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + i;
            const uint8_t l = blk[e / 2];
            const int lo = (e & 1) ? (l >> 4) : (l & 0x0F);
            const int hi = (blk[128 + e / 4] >> (2 * (e % 4))) & 0x03;
            w[i] = scale * (float)((lo | (hi << 4)) - 32);
        }
    }
}

}  // namespace jinf
