// Exposes the reference's own CPU routines (compiled from
// /root/reference/src/quant.cpp where it lies) under C names, so the oracle's
// restatement can be checked against them.  Test infrastructure only.
#include "jinf/quant.h"

extern "C" void jref_dequantize_q4_0(const void* blocks, float* out, int n_blocks) {
    jinf_dequantize_q4_0(static_cast<const jinf_block_q4_0*>(blocks), out, n_blocks);
}

// The reference's fp16 -> fp32 conversion, reached through its generic
// dispatcher (src/quant.cpp:108-136, JINF_TYPE_F16 branch).
extern "C" void jref_f16_to_f32(const void* halfs, float* out, long long n) {
    jinf_dequantize(halfs, JINF_TYPE_F16, out, (int64_t)n);
}

extern "C" void jref_dequantize_q4_K(const void* blocks, float* out, int n_blocks) {
    jinf_dequantize_q4_K(static_cast<const jinf_block_q4_K*>(blocks), out, n_blocks);
}

extern "C" void jref_dequantize_q8_0(const void* blocks, float* out, int n_blocks) {
    jinf_dequantize_q8_0(static_cast<const jinf_block_q8_0*>(blocks), out, n_blocks);
}
