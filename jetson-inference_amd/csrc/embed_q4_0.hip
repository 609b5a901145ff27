// GGUF Q4_0 token-embedding gather + dequant for gfx950.
//
// Semantics (reference src/engine.cpp:311-317 row addressing,
// cuda/dequant_kernels.cu:6-21 and src/quant.cpp:49-60 block decode):
//   row   = table + id * (n_embd/32) * 18 bytes
//   block b of the row = { uint16 d (binary16), uint8 qs[16] }
//   out[32b + 2j]     = ((qs[j] & 15) - 8) * d
//   out[32b + 2j + 1] = ((qs[j] >> 4) - 8) * d
// The product of an integer in [-8, 7] and a binary16 scale is exact in fp32,
// so the fp32 output is exact and the fp16 output is one RNE rounding of the
// exact value: both are bit-exact by construction.
//
// Design: grid = (ids, row segments).  A segment (<= kSegBlocks blocks) of
// the quantized row is staged into LDS with the widest load the row's
// alignment allows (16 bytes for Llama rows: 2304 = 144 * 16), because the
// 18-byte blocks are not 16-byte aligned individually.  Each lane then
// decodes one output unit of 16 bytes (8 fp16 or 4 fp32 values) from the
// block's scale and 4 (or 2) nibble bytes read from LDS, and consecutive
// lanes store consecutive 16-byte units, so stores are fully coalesced.
// fp16 decode is exact and packed: 0x6400 | nibble is the binary16 value
// 1024 + nibble; subtracting 1032 gives nibble - 8 exactly, and one packed
// binary16 multiply by d is the single RNE rounding of the exact product
// (fp16 denormals are preserved by the default MODE).
// Ids outside [0, n_vocab) produce +0.0 rows and read nothing.
#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"

namespace jinf {

constexpr int kSegBlocks = 512;  // blocks per workgroup (9216 bytes of LDS)
constexpr int kQ4Bytes = 18;

template <int LW> struct Word;
template <> struct Word<16> { typedef uint4 T; };
template <> struct Word<4> { typedef uint32_t T; };
template <> struct Word<2> { typedef uint16_t T; };
template <> struct Word<1> { typedef uint8_t T; };

// Four nibble bytes (little-endian in w) -> 8 binary16 values in jinf order,
// each = (nibble - 8) * d rounded once.
__device__ __forceinline__ uint4 decode8_f16(uint32_t w, uint16_t d) {
    const uint32_t p0 = (w & 0xFu) | ((w & 0xF0u) << 12);
    const uint32_t p1 = ((w >> 8) & 0xFu) | ((w & 0xF000u) << 4);
    const uint32_t p2 = ((w >> 16) & 0xFu) | ((w >> 4) & 0xF0000u);
    const uint32_t p3 = ((w >> 24) & 0xFu) | ((w >> 12) & 0xF0000u);
    const half2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    const _Float16 dh = __builtin_bit_cast(_Float16, d);
    const half2v dd = {dh, dh};
    uint32_t r[4];
    const uint32_t p[4] = {p0, p1, p2, p3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        half2v h = __builtin_bit_cast(half2v, p[i] | 0x64006400u);
        h = h - bias;  // exact: nibble - 8
        h = h * dd;    // single RNE rounding of the exact product
        r[i] = __builtin_bit_cast(uint32_t, h);
    }
    return make_uint4(r[0], r[1], r[2], r[3]);
}

// Two nibble bytes (low 16 bits of w) -> 4 fp32 values, exact.
__device__ __forceinline__ float4 decode4_f32(uint32_t w, uint16_t d) {
    const float df = h2f(d);
    return make_float4((float)((int)(w & 0xFu) - 8) * df,
                       (float)((int)((w >> 4) & 0xFu) - 8) * df,
                       (float)((int)((w >> 8) & 0xFu) - 8) * df,
                       (float)((int)((w >> 12) & 0xFu) - 8) * df);
}

// VST: output rows are 16-byte aligned, so each unit is one 16-byte store;
// otherwise each value is stored separately.
template <typename TO, int VST>
__device__ __forceinline__ void store_unit(TO* p, uint4 bits) {
    if constexpr (VST) {
        *reinterpret_cast<uint4*>(p) = bits;
    } else {
        const uint32_t w[4] = {bits.x, bits.y, bits.z, bits.w};
        if constexpr (sizeof(TO) == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) reinterpret_cast<uint32_t*>(p)[i] = w[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                reinterpret_cast<uint16_t*>(p)[2 * i] = (uint16_t)(w[i] & 0xFFFFu);
                reinterpret_cast<uint16_t*>(p)[2 * i + 1] = (uint16_t)(w[i] >> 16);
            }
        }
    }
}

template <typename TO, int LW, int VST>
__global__ __launch_bounds__(256) void embed_q4_0_kernel(
    TO* out, int64_t ld_out, const uint8_t* table, int n_vocab, int nb_row,
    const int32_t* ids) {
    // Output unit: 16 bytes = 8 fp16 or 4 fp32 values; kUPB units per block.
    constexpr int kVals = 16 / (int)sizeof(TO);
    constexpr int kUPB = 32 / kVals;
    __shared__ uint16_t lds[kSegBlocks * kQ4Bytes / 2];
    const int64_t r = blockIdx.x;
    const int b0 = blockIdx.y * kSegBlocks;
    const int nbs = min(kSegBlocks, nb_row - b0);
    const int nunits = nbs * kUPB;
    TO* orow = out + r * ld_out + (int64_t)b0 * 32;
    const int id = ids ? ids[r] : (int)r;
    if (id < 0 || id >= n_vocab) {
        for (int u = threadIdx.x; u < nunits; u += blockDim.x)
            store_unit<TO, VST>(orow + (int64_t)u * kVals, make_uint4(0, 0, 0, 0));
        return;
    }
    typedef typename Word<LW>::T W;
    const W* src = reinterpret_cast<const W*>(
        table + ((int64_t)id * nb_row + b0) * kQ4Bytes);
    W* dst = reinterpret_cast<W*>(lds);
    const int nw = nbs * kQ4Bytes / LW;
    for (int i = threadIdx.x; i < nw; i += blockDim.x) dst[i] = src[i];
    __syncthreads();
    for (int u = threadIdx.x; u < nunits; u += blockDim.x) {
        const int b = u / kUPB;
        const int q = u % kUPB;
        const int hb = b * (kQ4Bytes / 2);  // block start in 16-bit words
        const uint16_t d = lds[hb];
        if constexpr (kVals == 8) {
            // nibble bytes 4q .. 4q+3 of qs: words hb+1+2q, hb+2+2q
            const uint32_t w = (uint32_t)lds[hb + 1 + 2 * q] | ((uint32_t)lds[hb + 2 + 2 * q] << 16);
            store_unit<TO, VST>(orow + (int64_t)u * kVals, decode8_f16(w, d));
        } else {
            // nibble bytes 2q, 2q+1 of qs: word hb+1+q
            const uint32_t w = lds[hb + 1 + q];
            store_unit<TO, VST>(orow + (int64_t)u * kVals,
                                __builtin_bit_cast(uint4, decode4_f32(w, d)));
        }
    }
}

template <typename TO, int VST>
static int embed_launch(void* out, int64_t ld_out, const void* table, int n_vocab, int n_embd,
                        const int32_t* ids, int n_ids, hipStream_t stream) {
    static_assert((kSegBlocks * kQ4Bytes) % 16 == 0, "segment must hold whole 16-byte words");
    const int nb_row = n_embd / 32;
    const int64_t row_bytes = (int64_t)nb_row * kQ4Bytes;
    const int segs = (nb_row + kSegBlocks - 1) / kSegBlocks;
    const int units = (nb_row < kSegBlocks ? nb_row : kSegBlocks) * (32 * (int)sizeof(TO) / 16);
    int bs = round_up(units, kWave);
    if (bs > 256) bs = 256;
    const dim3 grid(n_ids, segs);
    TO* o = static_cast<TO*>(out);
    const uint8_t* t = static_cast<const uint8_t*>(table);
    // Widest staging word that keeps every segment start aligned (segment
    // starts are multiples of 512 blocks = 9216 bytes).
    if (aligned(table, 16) && row_bytes % 16 == 0)
        return launch(embed_q4_0_kernel<TO, 16, VST>, grid, dim3(bs), 0, stream, o, ld_out, t,
                      n_vocab, nb_row, ids);
    if (aligned(table, 4) && row_bytes % 4 == 0)
        return launch(embed_q4_0_kernel<TO, 4, VST>, grid, dim3(bs), 0, stream, o, ld_out, t,
                      n_vocab, nb_row, ids);
    if (aligned(table, 2))
        return launch(embed_q4_0_kernel<TO, 2, VST>, grid, dim3(bs), 0, stream, o, ld_out, t,
                      n_vocab, nb_row, ids);
    return launch(embed_q4_0_kernel<TO, 1, VST>, grid, dim3(bs), 0, stream, o, ld_out, t,
                  n_vocab, nb_row, ids);
}

static int embed_dispatch(void* out, int64_t ld_out, const void* table, int n_vocab, int n_embd,
                          const int32_t* ids, int n_ids, int out_type, hipStream_t stream) {
    if (n_ids < 0 || n_embd < 0 || n_vocab < 0) return JINF_HIP_ERR_INVALID;
    if (n_ids == 0 || n_embd == 0) return JINF_HIP_OK;
    if (n_embd % 32 != 0 || !out || !table || ld_out < n_embd) return JINF_HIP_ERR_INVALID;
    if (!ids && n_ids > n_vocab) return JINF_HIP_ERR_INVALID;
    if (out_type != JINF_HIP_F16 && out_type != JINF_HIP_F32) return JINF_HIP_ERR_INVALID;
    const int64_t osz = out_type == JINF_HIP_F16 ? 2 : 4;
    if (!aligned(out, osz)) return JINF_HIP_ERR_INVALID;
    if ((n_embd + kSegBlocks * 32 - 1) / (kSegBlocks * 32) > 65535) return JINF_HIP_ERR_INVALID;
    const bool vst = aligned(out, 16) && (ld_out * osz) % 16 == 0;
    if (out_type == JINF_HIP_F16)
        return vst ? embed_launch<uint16_t, 1>(out, ld_out, table, n_vocab, n_embd, ids, n_ids,
                                               stream)
                   : embed_launch<uint16_t, 0>(out, ld_out, table, n_vocab, n_embd, ids, n_ids,
                                               stream);
    return vst ? embed_launch<float, 1>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, stream)
               : embed_launch<float, 0>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, stream);
}

}  // namespace jinf

extern "C" int jinf_embed_q4_0(void* out, int ld_out, const void* table, int n_vocab, int n_embd,
                               const int32_t* ids, int n_ids, int out_type, hipStream_t stream) {
    return jinf::embed_dispatch(out, ld_out, table, n_vocab, n_embd, ids, n_ids, out_type,
                                stream);
}

// Drop-in for cuda/dequant_kernels.cu:116-122: n_blocks consecutive blocks
// (one "row" of 32*n_blocks values) to fp32.
extern "C" void jinf_cuda_dequantize_q4_0(const void* data, float* output, int n_blocks,
                                          hipStream_t stream) {
    if (n_blocks <= 0) return;
    if (n_blocks > (int)(0x7FFFFFFF / 32)) {
        JINF_LOG("jinf_cuda_dequantize_q4_0: n_blocks=%d too large", n_blocks);
        return;
    }
    const int st = jinf::embed_dispatch(output, (int64_t)n_blocks * 32, data, 1, n_blocks * 32,
                                        nullptr, 1, JINF_HIP_F32, stream);
    if (st == JINF_HIP_ERR_INVALID)
        JINF_LOG("jinf_cuda_dequantize_q4_0: invalid argument (n_blocks=%d)", n_blocks);
}
