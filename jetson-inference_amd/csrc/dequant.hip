// Gather + dequantize rows of GGUF block tables for Q8_0, Q4_K and Q6_K
// (Q4_0 has its own bandwidth-tuned kernel in embed_q4_0.hip), and the
// reference's per-row dequant launchers for those formats.
//
// Semantics (reference cuda/dequant_kernels.cu:25-110, :124-146; the
// engine's per-type embedding dispatch src/engine.cpp:311-334): row ids[i] of
// a table of n_vocab rows of n_embd values is dequantized to fp32 (or rounded
// once to fp16).  Weights are bit-identical to the reference's (decode8 in
// quant_device.h).  An id outside [0, n_vocab) gives a +0.0 row (the reference
// does not check ids).
//
// One lane per 8 consecutive values: it decodes them from the block with byte
// loads (any alignment) and writes them with 16-byte stores when the output
// rows are 16-byte aligned.  These calls move one row per token in the
// engine, so they sit at the launch-latency floor; the layout keeps them
// coalesced anyway.
#include "jinf_device.h"
#include "jinf_host.h"
#include "quant_device.h"
#include "jinf/kernels.h"
#include "jinf/kernels_ext.h"

namespace jinf {

constexpr int kDqBlock = 256;

template <typename TO, bool VEC>
__device__ __forceinline__ void store8(TO* p, const float (&w)[8]) {
    if constexpr (sizeof(TO) == 4) {
        if constexpr (VEC) {
            reinterpret_cast<float4*>(p)[0] = make_float4(w[0], w[1], w[2], w[3]);
            reinterpret_cast<float4*>(p)[1] = make_float4(w[4], w[5], w[6], w[7]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) p[i] = w[i];
        }
    } else {
        const uint32_t h0 = f2h2(w[0], w[1]), h1 = f2h2(w[2], w[3]);
        const uint32_t h2 = f2h2(w[4], w[5]), h3 = f2h2(w[6], w[7]);
        if constexpr (VEC) {
            *reinterpret_cast<uint4*>(p) = make_uint4(h0, h1, h2, h3);
        } else {
            const uint32_t hs[4] = {h0, h1, h2, h3};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[2 * i] = (uint16_t)(hs[i] & 0xFFFFu);
                p[2 * i + 1] = (uint16_t)(hs[i] >> 16);
            }
        }
    }
}

// grid: (n_ids, ceil(n_embd / 8 / 256)); lane = one 8-value group of a row.
template <int QT, typename TO, bool VEC>
__global__ __launch_bounds__(kDqBlock) void dequant_rows_kernel(
    TO* __restrict__ out, int64_t ld_out, const uint8_t* __restrict__ table, int64_t row_bytes,
    int n_vocab, int n_groups, const int32_t* __restrict__ ids) {
    constexpr int E = QGeom<QT>::kElems, B = QGeom<QT>::kBytes;
    const int i = blockIdx.x;
    const int gi = blockIdx.y * kDqBlock + threadIdx.x;
    if (gi >= n_groups) return;
    const int64_t id = ids ? (int64_t)ids[i] : (int64_t)i;
    float w[8];
    if (id < 0 || id >= n_vocab) {
#pragma unroll
        for (int k = 0; k < 8; ++k) w[k] = 0.0f;
    } else {
        decode8<QT>(table + id * row_bytes + (int64_t)(gi / (E / 8)) * B, (gi % (E / 8)) * 8, w);
    }
    store8<TO, VEC>(out + (int64_t)i * ld_out + 8 * (int64_t)gi, w);
}

template <int QT, typename TO>
static int dq_launch(void* out, int64_t ld_out, const void* table, int n_vocab, int n_embd,
                     const int32_t* ids, int n_ids, hipStream_t stream) {
    constexpr int E = QGeom<QT>::kElems, B = QGeom<QT>::kBytes;
    const int n_groups = n_embd / 8;
    const dim3 grid(n_ids, (n_groups + kDqBlock - 1) / kDqBlock);
    const int64_t row_bytes = (int64_t)(n_embd / E) * B;
    TO* o = static_cast<TO*>(out);
    const uint8_t* t = static_cast<const uint8_t*>(table);
    if (aligned(out, 16) && (ld_out * (int64_t)sizeof(TO)) % 16 == 0)
        return launch(dequant_rows_kernel<QT, TO, true>, grid, dim3(kDqBlock), 0, stream, o,
                      ld_out, t, row_bytes, n_vocab, n_groups, ids);
    return launch(dequant_rows_kernel<QT, TO, false>, grid, dim3(kDqBlock), 0, stream, o, ld_out,
                  t, row_bytes, n_vocab, n_groups, ids);
}

template <int QT>
static int dq_pick(void* out, int64_t ld_out, const void* table, int n_vocab, int n_embd,
                   const int32_t* ids, int n_ids, int out_type, hipStream_t stream) {
    if (out_type == JINF_HIP_F16)
        return dq_launch<QT, uint16_t>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, stream);
    return dq_launch<QT, float>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, stream);
}

static int dequant_rows(void* out, int64_t ld_out, const void* table, int qtype, int n_vocab,
                        int n_embd, const int32_t* ids, int n_ids, int out_type,
                        hipStream_t stream) {
    int elems;
    switch (qtype) {
        case kQ4_0: case kQ8_0: elems = 32; break;
        case kQ4_K: case kQ6_K: elems = 256; break;
        default: return JINF_HIP_ERR_INVALID;
    }
    if (n_ids < 0 || n_embd < 0 || n_vocab < 0) return JINF_HIP_ERR_INVALID;
    if (n_ids == 0 || n_embd == 0) return JINF_HIP_OK;
    if (n_embd % elems != 0 || !out || !table || ld_out < n_embd) return JINF_HIP_ERR_INVALID;
    if (!ids && n_ids > n_vocab) return JINF_HIP_ERR_INVALID;
    if (out_type != JINF_HIP_F16 && out_type != JINF_HIP_F32) return JINF_HIP_ERR_INVALID;
    if (!aligned(out, out_type == JINF_HIP_F16 ? 2 : 4)) return JINF_HIP_ERR_INVALID;
    if ((int64_t)n_embd / 8 > 65535LL * kDqBlock) return JINF_HIP_ERR_INVALID;
    if (qtype == kQ4_0) {
        if (ld_out > 0x7FFFFFFF) return JINF_HIP_ERR_INVALID;
        return jinf_embed_q4_0(out, (int)ld_out, table, n_vocab, n_embd, ids, n_ids, out_type,
                               stream);
    }
    switch (qtype) {
        case kQ8_0: return dq_pick<kQ8_0>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, out_type, stream);
        case kQ4_K: return dq_pick<kQ4_K>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, out_type, stream);
        default: return dq_pick<kQ6_K>(out, ld_out, table, n_vocab, n_embd, ids, n_ids, out_type, stream);
    }
}

// The reference's per-row launchers: n_blocks consecutive blocks -> fp32.
template <int QT>
static void dequant_drop_in(const char* name, const void* data, float* output, int n_blocks,
                            hipStream_t stream) {
    constexpr int E = QGeom<QT>::kElems;
    if (n_blocks <= 0) return;
    if (n_blocks > 0x7FFFFFFF / E) {
        JINF_LOG("%s: n_blocks=%d too large", name, n_blocks);
        return;
    }
    const int st = dequant_rows(output, (int64_t)n_blocks * E, data, QT, 1, n_blocks * E,
                                nullptr, 1, JINF_HIP_F32, stream);
    if (st == JINF_HIP_ERR_INVALID) JINF_LOG("%s: invalid argument (n_blocks=%d)", name, n_blocks);
}

}  // namespace jinf

extern "C" int jinf_dequant_rows(void* out, int ld_out, const void* table, int qtype, int n_vocab,
                                 int n_embd, const int32_t* ids, int n_ids, int out_type,
                                 hipStream_t stream) {
    return jinf::dequant_rows(out, ld_out, table, qtype, n_vocab, n_embd, ids, n_ids, out_type,
                              stream);
}

// Drop-ins for cuda/dequant_kernels.cu:124-146.
extern "C" void jinf_cuda_dequantize_q4_K(const void* data, float* output, int n_blocks,
                                          hipStream_t stream) {
    jinf::dequant_drop_in<jinf::kQ4_K>("jinf_cuda_dequantize_q4_K", data, output, n_blocks, stream);
}

extern "C" void jinf_cuda_dequantize_q8_0(const void* data, float* output, int n_blocks,
                                          hipStream_t stream) {
    jinf::dequant_drop_in<jinf::kQ8_0>("jinf_cuda_dequantize_q8_0", data, output, n_blocks, stream);
}

extern "C" void jinf_cuda_dequantize_q6_K(const void* data, float* output, int n_blocks,
                                          hipStream_t stream) {
    jinf::dequant_drop_in<jinf::kQ6_K>("jinf_cuda_dequantize_q6_K", data, output, n_blocks, stream);
}
