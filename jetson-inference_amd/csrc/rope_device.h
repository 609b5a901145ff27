// Interleaved RoPE arithmetic shared by the RoPE kernels and the fused
// projection GEMVs (reference cuda/rope_kernel.cu:8-50):
//   theta_i = fl32(base ^ (-2i / head_dim)),   a = fl32((float)pos * theta_i)
//   c, s    = fl32(cos a), fl32(sin a)        (evaluated in fp64, rounded once)
//   x0' = x0*c - x1*s,  x1' = x0*s + x1*c      (every product and sum in fp32)
#pragma once

#include <math.h>

#include "jinf_device.h"

namespace jinf {

constexpr int kRopeMaxHalf = 256;  // head_dim <= 512

// theta_i for i < head_dim / 2, passed to kernels by value.  Kernels for
// head_dim <= 128 take the 64-entry form: a smaller kernel-argument block is
// cheaper to dispatch.
template <int N>
struct RopeThetaN {
    float t[N];
};
using RopeTheta = RopeThetaN<kRopeMaxHalf>;
using RopeTheta64 = RopeThetaN<64>;

__device__ __forceinline__ void rot(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c - x1 * s;
    const float b = x0 * s + x1 * c;
    x0 = a;
    x1 = b;
}

// (cos a, sin a) of an fp32 angle, evaluated in fp64 and rounded once to
// fp32.  For |a| < 2^20:
//   - reduction a = k (pi/2) + r with k = rint(a * 2/pi) and pi/2 split
//     Cody-Waite style into P1 + P2 + P3 (P1, P2 the leading two 33-bit
//     chunks of pi/2, so k * P1 and k * P2 are exact for |k| < 2^20, and
//     a - k * P1 is exact by Sterbenz; P3 the next 53 bits).  The error of r
//     is a few fp64 ulps of r plus |k| * 2^-119;
//   - sin r and cos r by their Taylor series through r^13 and r^14 on
//     |r| <= pi/4 (truncation below |r|^15/15! < 2.1e-14 and
//     |r|^16/16! < 1.1e-15), Horner in fp64;
//   - the quadrant k mod 4 selects and negates.
// The fp64 result is within ~1e-14 of the true value, so the fp32 rounding is
// the correctly rounded cos / sin except when the true value lies that close
// to a rounding midpoint.  Larger |a| (and NaN) take the device library's fp64
// sincos.  About 25 fp64 operations with no branch in the common case.
__device__ __forceinline__ float2 cos_sin_f32(float a) {
    if (!(fabsf(a) < 0x1p20f)) {
        double sn, cn;
        sincos((double)a, &sn, &cn);
        return make_float2((float)cn, (float)sn);
    }
    const double x = (double)a;
    const double k = rint(x * 0x1.45f306dc9c883p-1);   // x * (2/pi)
    double r = fma(-k, 0x1.921fb54400000p+0, x);        // P1
    r = fma(-k, 0x1.0b4611a600000p-34, r);               // P2
    r = fma(-k, 0x1.3198a2e037073p-69, r);               // P3
    const double z = r * r;
    double ps = 1.0 / 6227020800.0;                      // 1/13!
    ps = fma(ps, z, -1.0 / 39916800.0);                  // -1/11!
    ps = fma(ps, z, 1.0 / 362880.0);                     // 1/9!
    ps = fma(ps, z, -1.0 / 5040.0);                      // -1/7!
    ps = fma(ps, z, 1.0 / 120.0);                        // 1/5!
    ps = fma(ps, z, -1.0 / 6.0);                         // -1/3!
    const double sn = fma(r * z, ps, r);
    double pc = -1.0 / 87178291200.0;                    // -1/14!
    pc = fma(pc, z, 1.0 / 479001600.0);                  // 1/12!
    pc = fma(pc, z, -1.0 / 3628800.0);                   // -1/10!
    pc = fma(pc, z, 1.0 / 40320.0);                      // 1/8!
    pc = fma(pc, z, -1.0 / 720.0);                       // -1/6!
    pc = fma(pc, z, 1.0 / 24.0);                         // 1/4!
    pc = fma(pc, z, -0.5);                               // -1/2!
    const double cn = fma(z, pc, 1.0);
    const int q = (int)(int64_t)k & 3;
    double c = (q & 1) ? sn : cn;
    double s = (q & 1) ? cn : sn;
    if (q == 1 || q == 2) c = -c;
    if (q >= 2) s = -s;
    return make_float2((float)c, (float)s);
}

// (cos, sin) of the RoPE angle fl32(pos * theta).
__device__ __forceinline__ float2 rope_cs(int pos, float theta) {
#pragma clang fp contract(off)
    const float a = (float)pos * theta;
    return cos_sin_f32(a);
}

// theta_i in fp64 from the exponent formed exactly as the reference forms it
// in fp32 (-2.0f * i / hd), rounded once: the correctly rounded power.
// Entries past head_dim / 2 (or past N) are zero / not written.
template <int N>
inline void theta_table(RopeThetaN<N>& th, int head_dim, float base) {
    const int half = head_dim / 2 < N ? head_dim / 2 : N;
    for (int i = 0; i < N; ++i) th.t[i] = 0.0f;
    for (int i = 0; i < half; ++i) {
        volatile float e = -2.0f * (float)i;
        e = e / (float)head_dim;
        th.t[i] = (float)pow((double)base, (double)e);
    }
}

}  // namespace jinf
