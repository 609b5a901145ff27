// Device-side helpers shared by the jinf gfx950 kernels: binary16 <-> binary32
// conversion, 16-byte vector access, and wave64 / workgroup reductions.
//
// Every reduction here is deterministic: partials are combined in a fixed
// order, so a kernel run twice on the same input gives identical bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jinf {

constexpr int kWave = 64;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Exact binary16 -> binary32 widening (subnormals, -0, Inf, NaN preserved);
// plays the role of half_to_float (reference cuda/cuda_utils.cuh:10-14).
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// binary32 -> binary16 with round-to-nearest-even (default MODE: RNE, fp16
// denormals kept).  The conversion is written as an explicit instruction so
// the compiler cannot merge it with the fp32 multiply or add that produced the
// value (it otherwise folds them into one v_fma_mix*_f16 with a +0 addend,
// which need not round through fp32 first and turns a -0 product into +0).
// Every stored fp16 value is thus fl16(fl32(expression)).
__device__ __forceinline__ uint16_t f2h(float f) {
    uint32_t r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(f));
    return (uint16_t)r;
}

// Two binary32 -> packed binary16 (lo in bits 0..15), RNE, same guarantee.
__device__ __forceinline__ uint32_t f2h2(float lo, float hi) {
    uint32_t r;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}

// 16-byte global access.  NT = true marks the access nontemporal (streamed
// data touched once per launch): measured on MI355X it raises copy bandwidth
// from ~4.8 to ~5.7 TB/s because the lines do not displace reusable ones in
// L2 / Infinity Cache.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p) {
    if constexpr (NT) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}

template <bool NT>
__device__ __forceinline__ void st16(void* p, uint4 v) {
    if constexpr (NT) {
        const u32x4 w = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
    } else {
        *reinterpret_cast<uint4*>(p) = v;
    }
}

// Storage traits: a "chunk" is one 16-byte vector of the storage type.
template <typename T> struct Act;

template <> struct Act<float> {
    static constexpr int kElems = 4;
    __device__ static __forceinline__ void unpack(uint4 x, float (&v)[4]) {
        v[0] = __builtin_bit_cast(float, x.x); v[1] = __builtin_bit_cast(float, x.y);
        v[2] = __builtin_bit_cast(float, x.z); v[3] = __builtin_bit_cast(float, x.w);
    }
    __device__ static __forceinline__ uint4 pack(const float (&v)[4]) {
        return make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                          __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
    }
    template <bool NT = true>
    __device__ static __forceinline__ void load(const float* p, float (&v)[4]) {
        unpack(ld16<NT>(p), v);
    }
    template <bool NT = true>
    __device__ static __forceinline__ void store(float* p, const float (&v)[4]) {
        st16<NT>(p, pack(v));
    }
    __device__ static __forceinline__ float load1(const float* p) { return *p; }
    __device__ static __forceinline__ void store1(float* p, float v) { *p = v; }
    // Round an fp32 value to the storage precision (identity for fp32).
    __device__ static __forceinline__ float round(float v) { return v; }
};

template <> struct Act<uint16_t> {
    static constexpr int kElems = 8;
    __device__ static __forceinline__ void unpack(uint4 x, float (&v)[8]) {
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = h2f((uint16_t)(w[i] & 0xFFFFu));
            v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
        }
    }
    __device__ static __forceinline__ uint4 pack(const float (&v)[8]) {
        return make_uint4(f2h2(v[0], v[1]), f2h2(v[2], v[3]), f2h2(v[4], v[5]),
                          f2h2(v[6], v[7]));
    }
    template <bool NT = true>
    __device__ static __forceinline__ void load(const uint16_t* p, float (&v)[8]) {
        unpack(ld16<NT>(p), v);
    }
    template <bool NT = true>
    __device__ static __forceinline__ void store(uint16_t* p, const float (&v)[8]) {
        st16<NT>(p, pack(v));
    }
    __device__ static __forceinline__ float load1(const uint16_t* p) { return h2f(*p); }
    __device__ static __forceinline__ void store1(uint16_t* p, float v) { *p = f2h(v); }
    __device__ static __forceinline__ float round(float v) { return h2f(f2h(v)); }
};

// Weight element read (fp32 or fp16 storage), widened exactly to fp32.
__device__ __forceinline__ float wload(const float* w, int i) { return w[i]; }
__device__ __forceinline__ float wload(const uint16_t* w, int i) { return h2f(w[i]); }

// ---- wave64 reductions (butterfly: every lane ends with the full result) ----

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// fp32 wave sum without LDS round trips: four DPP steps (quad swaps, then
// rotations by 4 and 8 lanes within each row of 16) leave every lane with its
// row's sum; the four row sums are read into scalars and added in row order.
// Returns the same value in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// v + (v of lane l ^ 32), in every lane, with one v_permlane32_swap: swapping
// v with itself leaves lanes l and l ^ 32's values in the two results' lane l.
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                     false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                     false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return ((r0 + r1) + r2) + r3;
}

// exp(a) for a softmax argument a = s - m <= 0 in two VALU ops: 2^fl(a*fl(log2 e))
// through v_exp_f32 (1 ulp).  The product's rounding and log2 e's shift the
// exponent by at most |a| * 1.05e-7, so the relative error is at most
// 7.3e-8 * |a| + 1.2e-7: below 6.5e-6 for every normal fp32 result (a above
// about -87.3); a Cody-Waite split of a*log2(e) into hi + lo with
// 2^hi * (1 + lo*ln2) would stay within about 2 ulp for four more operations.
// -inf gives +0; subnormal results may flush to 0 (absolute error < 1.2e-38).
__device__ __forceinline__ float exp_neg_fast(float a) {
    return __builtin_amdgcn_exp2f(a * 1.44269502162933349609375f);
}

// fp64 wave sum, same DPP pattern as wave_sum_f32 (both halves of each value
// moved by DPP; the four row sums added in row order).  Every lane gets the
// result.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<0xB1>(v);
    v += dpp_f64<0x4E>(v);
    v += dpp_f64<0x124>(v);
    v += dpp_f64<0x128>(v);
    double r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t u = __double_as_longlong(v);
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, 16 * i);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 16 * i);
        r[i] = __longlong_as_double((int64_t)(((uint64_t)hi << 32) | lo));
    }
    return ((r[0] + r[1]) + r[2]) + r[3];
}

// fp32 wave max, same DPP pattern as wave_sum_f32 (every lane gets the result).
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x124>(v));
    v = fmaxf(v, dpp_f32<0x128>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Workgroup reductions.  blockDim.x must be a multiple of 64 and at most 1024.
// `lds` holds one slot per wave; each thread folds the per-wave partials in
// wave order, so every thread returns the same value without a second
// barrier.  A trailing barrier makes `lds` safe to reuse by the caller.
__device__ __forceinline__ double block_sum(double v, double* lds) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    const int nw = blockDim.x / kWave;
    double s = lds[0];
    for (int i = 1; i < nw; ++i) s += lds[i];
    __syncthreads();
    return s;
}

// RMSNorm scale rs = 1/sqrt(fl32(fl32(ss)/n) + eps) from an fp64 sum of
// squares; the sqrt and divide in fp64, rounded once to fp32.
__device__ __forceinline__ float rms_scale(double ss, int n, float eps) {
#pragma clang fp contract(off)
    const float m = (float)ss / (float)n;
    const float t = m + eps;
    return (float)(1.0 / sqrt((double)t));
}

// SwiGLU in fp32 as the reference writes it (cuda/silu_kernel.cu:6-18):
// (g / (1 + expf(-g))) * u, no contraction.
__device__ __forceinline__ float swiglu_exact(float g, float u) {
#pragma clang fp contract(off)
    return (g / (1.0f + expf(-g))) * u;
}

__device__ __forceinline__ float block_max(float v, float* lds) {
    v = wave_max(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    const int nw = blockDim.x / kWave;
    float m = lds[0];
    for (int i = 1; i < nw; ++i) m = fmaxf(m, lds[i]);
    __syncthreads();
    return m;
}

// Device-coherent (sc1) record store / load for the cross-workgroup merge.
__device__ __forceinline__ void rec_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float rec_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One 16-byte direct-to-LDS load per lane: lane l's 16 bytes from gptr land
// at LDS byte lds_base + 16 l (lds_base wave-uniform).  Issued from inline
// assembly so that the compiler's wait-count tracking, which cannot tell
// this wave's K and V regions apart, adds no wait for it; the kernel waits
// for these loads itself (an uncounted load can only make the compiler's
// own waits longer, never shorter).
// M0 (the LDS destination register) is saved and restored around the load,
// so the statement leaves every register the compiler knows about intact.
__device__ __forceinline__ void lds_load16(const void* gptr, const void* lds_base) {
    const uint32_t off = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_base;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(gptr), "s"(__builtin_amdgcn_readfirstlane(off))
        : "memory");
}

// The same through a buffer resource: lane l's 16 bytes at byte offset
// voff + soff of the resource land at lds_base + 16 l.  soff is wave-uniform,
// so a caller that keeps each lane's voff from one tile to the next pays no
// vector arithmetic per load; bytes at or past the resource's num_records
// read as zero (no memory access).
__device__ __forceinline__ void lds_load16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff,
                                               const void* lds_base) {
    const uint32_t off = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_base;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "buffer_load_dwordx4 %1, %2, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(off)),
          "s"(__builtin_amdgcn_readfirstlane(soff))
        : "memory");
}

// s_waitcnt immediate that waits until at most N vector-memory operations
// are outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt and
// lgkmcnt left at their maxima).
template <int N>
constexpr int waitcnt_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    return (N & 0xF) | ((N >> 4) << 14) | 0x0F70;
}

}  // namespace jinf
