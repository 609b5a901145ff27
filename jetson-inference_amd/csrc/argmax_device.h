// Greedy argmax helpers shared by the decode engines: the reference's scan
// of the logits keeping strict improvements (src/engine.cpp:783-791).
#pragma once

#include "jinf_device.h"

namespace jinf {

constexpr int kArgThreads = 256;

// (bv, bi) <- (v, i) if v is larger, or equal with a smaller index.  A NaN v
// is never taken, and bv never becomes NaN.
__device__ __forceinline__ void take(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Workgroup-wide best (value, index) into thread 0.
__device__ __forceinline__ void block_best(float& bv, int& bi) {
    __shared__ float sv[kArgThreads / kWave];
    __shared__ int si[kArgThreads / kWave];
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        take(bv, bi, ov, oi);
    }
    const int w = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < kArgThreads / kWave; ++k) take(bv, bi, sv[k], si[k]);
}

}  // namespace jinf
