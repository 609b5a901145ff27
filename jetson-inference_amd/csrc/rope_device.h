// Interleaved RoPE arithmetic shared by the RoPE kernels and the fused
// projection GEMV (reference cuda/rope_kernel.cu:8-50):
//   theta_i = fl32(base ^ (-2i / head_dim)),   a = fl32((float)pos * theta_i)
//   c, s    = fl32(cos a), fl32(sin a)        (evaluated in fp64, rounded once)
//   x0' = x0*c - x1*s,  x1' = x0*s + x1*c      (every product and sum in fp32)
#pragma once

#include <math.h>

#include "jinf_device.h"

namespace jinf {

constexpr int kRopeMaxHalf = 256;  // head_dim <= 512

// theta_i for i < head_dim / 2, passed to kernels by value.
struct RopeTheta {
    float t[kRopeMaxHalf];
};

__device__ __forceinline__ void rot(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c - x1 * s;
    const float b = x0 * s + x1 * c;
    x0 = a;
    x1 = b;
}

// (cos, sin) of fl32(pos * theta), computed in fp64 and rounded to fp32: the
// correctly rounded values of the exact fp32 angle.
__device__ __forceinline__ float2 rope_cs(int pos, float theta) {
#pragma clang fp contract(off)
    const float a = (float)pos * theta;
    double sn, cn;
    sincos((double)a, &sn, &cn);
    return make_float2((float)cn, (float)sn);
}

// theta_i in fp64 from the exponent formed exactly as the reference forms it
// in fp32 (-2.0f * i / hd), rounded once: the correctly rounded power.
inline void theta_table(RopeTheta& th, int head_dim, float base) {
    const int half = head_dim / 2;
    for (int i = 0; i < kRopeMaxHalf; ++i) th.t[i] = 0.0f;
    for (int i = 0; i < half; ++i) {
        volatile float e = -2.0f * (float)i;
        e = e / (float)head_dim;
        th.t[i] = (float)pow((double)base, (double)e);
    }
}

}  // namespace jinf
