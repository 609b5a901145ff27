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
// Design: one lane per 16-byte output unit (8 fp16 or 4 fp32 values, a quarter
// or an eighth of a block); grid = (ids, unit tiles of a row).  Each lane reads
// its block's scale and its 4 (or 2) nibble bytes straight from global memory
// with 16-bit loads (blocks are 18 bytes, so every field is 2-byte aligned but
// not 4-byte aligned).  The 16 lanes that share a 288-byte run of blocks hit
// the same cache lines, so HBM sees each table byte once; consecutive lanes
// store consecutive 16-byte units with nontemporal stores, fully coalesced.
// Measured on MI355X (4096 ids of a 128256 x 4096 table -> fp16): 7.86 us with
// 256-lane workgroups (two per 4096-wide row), 8.1 us with 512 lanes, 8.3 us for
// staging the row through LDS first; 2 or 4 units per lane gain nothing.
// fp16 decode is exact and packed: 0x6400 | nibble is the binary16 value
// 1024 + nibble; subtracting 1032 gives nibble - 8 exactly, and one packed
// binary16 multiply by d is the single RNE rounding of the exact product
// (fp16 denormals are preserved by the default MODE).
// Ids outside [0, n_vocab) produce +0.0 rows and read nothing.
#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"

namespace jinf {

constexpr int kQ4Bytes = 18;
constexpr int kEmbedBlock = 256;

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
__device__ __forceinline__ uint4 decode4_f32(uint32_t w, uint16_t d) {
    const float df = h2f(d);
    const float v[4] = {(float)((int)(w & 0xFu) - 8) * df, (float)((int)((w >> 4) & 0xFu) - 8) * df,
                        (float)((int)((w >> 8) & 0xFu) - 8) * df,
                        (float)((int)((w >> 12) & 0xFu) - 8) * df};
    return Act<float>::pack(v);
}

// 16-bit little-endian field at an even byte offset (A2) or at any offset.
template <bool A2>
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    if constexpr (A2)
        return *reinterpret_cast<const uint16_t*>(p);
    else
        return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// VST: output rows are 16-byte aligned, so each unit is one 16-byte store;
// otherwise each value is stored separately.
template <typename TO, bool VST>
__device__ __forceinline__ void store_unit(TO* p, uint4 bits) {
    if constexpr (VST) {
        st16<true>(p, bits);
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

template <typename TO, bool A2, bool VST>
__global__ __launch_bounds__(kEmbedBlock) void embed_q4_0_kernel(
    TO* out, int64_t ld_out, const uint8_t* table, int n_vocab, int nb_row,
    const int32_t* ids) {
    // Output unit: 16 bytes = 8 fp16 or 4 fp32 values; kUPB units per block.
    constexpr int kVals = 16 / (int)sizeof(TO);
    constexpr int kUPB = 32 / kVals;
    const int64_t r = blockIdx.x;
    const int u = blockIdx.y * blockDim.x + threadIdx.x;
    if (u >= nb_row * kUPB) return;
    const int id = ids ? ids[r] : (int)r;
    TO* dst = out + r * ld_out + (int64_t)u * kVals;
    if (id < 0 || id >= n_vocab) {
        store_unit<TO, VST>(dst, make_uint4(0, 0, 0, 0));
        return;
    }
    const int b = u / kUPB;
    const int q = u % kUPB;
    const uint8_t* blk = table + ((int64_t)id * nb_row + b) * kQ4Bytes;
    const uint16_t d = (uint16_t)ld_u16<A2>(blk);
    if constexpr (kVals == 8) {
        // nibble bytes 4q .. 4q+3 of qs
        const uint32_t w = ld_u16<A2>(blk + 2 + 4 * q) | (ld_u16<A2>(blk + 4 + 4 * q) << 16);
        store_unit<TO, VST>(dst, decode8_f16(w, d));
    } else {
        // nibble bytes 2q, 2q+1 of qs
        store_unit<TO, VST>(dst, decode4_f32(ld_u16<A2>(blk + 2 + 2 * q), d));
    }
}

template <typename TO, bool A2, bool VST>
static int embed_launch(void* out, int64_t ld_out, const void* table, int n_vocab, int n_embd,
                        const int32_t* ids, int n_ids, hipStream_t stream) {
    const int nb_row = n_embd / 32;
    const int units = nb_row * (32 * (int)sizeof(TO) / 16);
    const int bs = units < kEmbedBlock ? round_up(units, kWave) : kEmbedBlock;
    const dim3 grid(n_ids, (units + bs - 1) / bs);
    return launch(embed_q4_0_kernel<TO, A2, VST>, grid, dim3(bs), 0, stream,
                  static_cast<TO*>(out), ld_out, static_cast<const uint8_t*>(table), n_vocab,
                  nb_row, ids);
}

template <typename TO>
static int embed_pick(void* out, int64_t ld_out, const void* table, int n_vocab, int n_embd,
                      const int32_t* ids, int n_ids, hipStream_t stream) {
    const bool vst = aligned(out, 16) && (ld_out * (int64_t)sizeof(TO)) % 16 == 0;
    const bool a2 = aligned(table, 2);
    if (vst)
        return a2 ? embed_launch<TO, true, true>(out, ld_out, table, n_vocab, n_embd, ids, n_ids,
                                                 stream)
                  : embed_launch<TO, false, true>(out, ld_out, table, n_vocab, n_embd, ids,
                                                  n_ids, stream);
    return a2 ? embed_launch<TO, true, false>(out, ld_out, table, n_vocab, n_embd, ids, n_ids,
                                              stream)
              : embed_launch<TO, false, false>(out, ld_out, table, n_vocab, n_embd, ids, n_ids,
                                               stream);
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
    // grid.y = unit tiles of one row (<= 65535)
    if ((int64_t)n_embd * osz / 16 > 65535LL * kEmbedBlock) return JINF_HIP_ERR_INVALID;
    if (out_type == JINF_HIP_F16)
        return embed_pick<uint16_t>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, stream);
    return embed_pick<float>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, stream);
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
