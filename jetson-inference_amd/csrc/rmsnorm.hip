// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Semantics (reference cuda/rmsnorm_kernel.cu:9-61, residual add
// cuda/matmul_kernels.cu:189-194, sequencing src/engine.cpp:466->487):
//   h_i  = x_i                      (plain norm), or
//   h_i  = round_act(r_i + x_i)     (fused; stored back to the residual)
//   ss   = sum_i h_i^2
//   rs   = 1 / sqrt(ss / n + eps)   (ss/n and +eps in fp32)
//   y_i  = round_act((h_i * rs) * w_i)
//
// Design: one workgroup per row.  The row is held in registers (up to
// kNormCPT 16-byte chunks per thread), so every input byte is read from HBM
// once and every output byte written once: the fused kernel moves 4 rows of
// traffic (r, x in; r', y out) instead of the reference's 3 + 2..3 rows for
// separate residual_add and rmsnorm launches.  The sum of squares is
// accumulated in fp64 (h_i^2 is exact in fp64), reduced across the wave by
// butterfly shuffles and across waves through LDS in a fixed order; 1/sqrt is
// evaluated in fp64 and rounded once.  The result is therefore independent of
// the launch shape and matches a sequential fp64 sum to within fp32 rounding.
// Rows longer than the register capacity, or not 16-byte aligned, take a
// two-pass loop kernel that re-reads the row.
#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"

namespace jinf {

constexpr int kNormCPT = 4;  // 16-byte chunks per thread held in registers

// E consecutive weight elements: raw bits loaded with the row or during the
// reduction's barrier (normal cached loads: every row re-reads the weight),
// widened to fp32 after the reduction.
template <typename TW, int E> struct WRaw {
    static constexpr int kWords = (E * (int)sizeof(TW) + 15) / 16;  // 16-byte words
    uint4 w[kWords];
};

template <int E>
__device__ __forceinline__ void wload_raw(const float* w, WRaw<float, E>& r) {
#pragma unroll
    for (int i = 0; i < WRaw<float, E>::kWords; ++i) r.w[i] = ld16<false>(w + 4 * i);
}
template <int E>
__device__ __forceinline__ void wload_raw(const uint16_t* w, WRaw<uint16_t, E>& r) {
    if constexpr (E == 8) {
        r.w[0] = ld16<false>(w);
    } else {
        const uint2 x = *reinterpret_cast<const uint2*>(w);
        r.w[0] = make_uint4(x.x, x.y, 0, 0);
    }
}
template <int E>
__device__ __forceinline__ void wunpack(const WRaw<float, E>& r, float (&v)[E]) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const uint4 q = r.w[i / 4];
        const uint32_t u = (i % 4 == 0) ? q.x : (i % 4 == 1) ? q.y : (i % 4 == 2) ? q.z : q.w;
        v[i] = __builtin_bit_cast(float, u);
    }
}
template <int E>
__device__ __forceinline__ void wunpack(const WRaw<uint16_t, E>& r, float (&v)[E]) {
    const uint32_t u[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
        v[2 * i] = h2f((uint16_t)(u[i] & 0xFFFFu));
        v[2 * i + 1] = h2f((uint16_t)(u[i] >> 16));
    }
}

// BS lanes (a template argument: with the block size known at compile time
// the chunk offsets are immediates), CPT chunks per lane.  WLATE issues the
// weight loads after the row's sum of squares, while the workgroup waits at
// its barrier: the weight is cache-resident (every row reads it), and keeping
// it out of the row's load phase shortens the critical path when a few rows
// each own a CU (64 rows of 8192: 3.40 -> 3.22 us measured, with CPT = 2).
// EXACT: the row is exactly BS * CPT chunks, so no chunk needs a bounds test.
// The tests put each chunk's loads inside a branch, after which the compiler
// waits for every outstanding load before the first store (64 rows of 8192:
// 3.93 us guarded against 3.22 us exact).
template <typename TA, typename TW, bool FUSED, int BS, int CPT, bool WLATE = false,
          bool EXACT = false>
__global__ __launch_bounds__(BS) void rmsnorm_vec_kernel(
    TA* out, int ld_out, TA* res, int ld_res, const TA* in, int ld_in,
    const TW* __restrict__ w, int n, float eps) {
#pragma clang fp contract(off)
    using A = Act<TA>;
    constexpr int E = A::kElems;
    __shared__ double red[16];
    const int64_t row = blockIdx.x;
    const int nch = n / E;
    constexpr int bs = BS;
    const TA* x = in + row * ld_in;
    TA* r = FUSED ? res + row * ld_res : nullptr;

    // The row stays in registers in its storage format (16-byte chunks); every
    // load is issued before any store (out may alias in).
    // The weight chunks are fetched with the row (WLATE: while the workgroup
    // waits at the reduction's barrier), so their latency is not paid again
    // after the reduction.
    uint4 hv[CPT];
    uint4 dv[CPT];
    WRaw<TW, E> wr[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (EXACT || c < nch) {
            if constexpr (FUSED) {
                hv[j] = ld16<true>(r + (int64_t)c * E);
                dv[j] = ld16<true>(x + (int64_t)c * E);
            } else {
                hv[j] = ld16<true>(x + (int64_t)c * E);
            }
            if constexpr (!WLATE) wload_raw<E>(w + c * E, wr[j]);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (EXACT || c < nch) {
            float h[E];
            A::unpack(hv[j], h);
            if constexpr (FUSED) {
                float d[E];
                A::unpack(dv[j], d);
#pragma unroll
                for (int e = 0; e < E; ++e) h[e] = h[e] + d[e];
                hv[j] = A::pack(h);  // the stored residual, rounded once
                st16<true>(r + (int64_t)c * E, hv[j]);
                A::unpack(hv[j], h);
            }
#pragma unroll
            for (int e = 0; e < E; ++e) ss = fma((double)h[e], (double)h[e], ss);
        }
    }
    // DPP wave sums, one LDS exchange and one barrier (`red` is not reused)
    ss = wave_sum_f64(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
    if constexpr (WLATE) {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = threadIdx.x + j * bs;
            if (EXACT || c < nch) wload_raw<E>(w + c * E, wr[j]);
        }
    }
    __syncthreads();
    ss = red[0];
#pragma unroll
    for (int i = 1; i < bs / kWave; ++i) ss += red[i];
    const float rs = rms_scale(ss, n, eps);
    TA* y = out + row * ld_out;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * bs;
        if (EXACT || c < nch) {
            float h[E], wv[E], o[E];
            A::unpack(hv[j], h);
            wunpack<E>(wr[j], wv);
#pragma unroll
            for (int e = 0; e < E; ++e) o[e] = (h[e] * rs) * wv[e];
            st16<true>(y + (int64_t)c * E, A::pack(o));
        }
    }
}

// Any length / alignment: pass 1 forms (and for the fused form stores) h and
// its sum of squares, pass 2 re-reads h and writes y.  Each element is read
// and written by the same thread in both passes, so in-place use is safe.
template <typename TA, typename TW, bool FUSED>
__global__ __launch_bounds__(1024) void rmsnorm_loop_kernel(
    TA* out, int ld_out, TA* res, int ld_res, const TA* in, int ld_in,
    const TW* __restrict__ w, int n, float eps) {
#pragma clang fp contract(off)
    using A = Act<TA>;
    __shared__ double red[16];
    const int64_t row = blockIdx.x;
    const TA* x = in + row * ld_in;
    TA* r = FUSED ? res + row * ld_res : nullptr;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = A::load1(x + i);
        if constexpr (FUSED) {
            v = A::round(A::load1(r + i) + v);
            A::store1(r + i, v);
        }
        ss = fma((double)v, (double)v, ss);
    }
    ss = block_sum(ss, red);
    const float rs = rms_scale(ss, n, eps);
    TA* y = out + row * ld_out;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = FUSED ? A::load1(r + i) : A::load1(x + i);
        A::store1(y + i, (v * rs) * wload(w, i));
    }
}

template <typename TA, typename TW, bool FUSED>
static int rmsnorm_launch(void* out, int ld_out, void* res, int ld_res, const void* in,
                          int ld_in, const void* w, int n_rows, int n, float eps,
                          hipStream_t stream) {
    constexpr int E = Act<TA>::kElems;
    constexpr int kVec = 16;
    const bool vec = (n % E == 0) && aligned(out, kVec) && aligned(in, kVec) &&
                     aligned(w, kVec) && ((int64_t)ld_out * sizeof(TA)) % kVec == 0 &&
                     ((int64_t)ld_in * sizeof(TA)) % kVec == 0 &&
                     (!FUSED || (aligned(res, kVec) && ((int64_t)ld_res * sizeof(TA)) % kVec == 0));
    const int nch = n / E;
    TA* o = static_cast<TA*>(out);
    TA* r = static_cast<TA*>(res);
    const TA* x = static_cast<const TA*>(in);
    const TW* wt = static_cast<const TW*>(w);
    // Few rows cannot fill 256 CUs, so each row's workgroup owns a CU and the
    // launch is latency-bound: two chunks per lane (all of a row's loads in
    // flight at once, half the waves of one chunk per lane), the weight
    // loaded late.  Measured at 64 rows of 8192 fp16: 1024 x 1 3.40 us,
    // 512 x 2 3.22 us, 256 x 4 3.30 us (each with the weight loaded late).
    // Splitting a row over several workgroups that exchange partial sums
    // through device-coherent memory was slower at every split (4.3 us at 2
    // workgroups per row, 10.4 us at 16): one exchange costs more than the
    // shorter per-CU load phase saves.
    if (vec && n_rows < 1024 && nch > 2 * kWave && nch <= 2 * 1024) {
        int bp = kWave;
        while (2 * bp < nch) bp *= 2;
        auto go = [&](auto kern) {
            return launch(kern, dim3(n_rows), dim3(bp), 0, stream, o, ld_out, r, ld_res, x,
                          ld_in, wt, n, eps);
        };
        const bool ex = nch == 2 * bp;
        switch (bp) {
            case 128: return ex ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 128, 2, true, true>)
                                : go(rmsnorm_vec_kernel<TA, TW, FUSED, 128, 2, true>);
            case 256: return ex ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 256, 2, true, true>)
                                : go(rmsnorm_vec_kernel<TA, TW, FUSED, 256, 2, true>);
            case 512: return ex ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 512, 2, true, true>)
                                : go(rmsnorm_vec_kernel<TA, TW, FUSED, 512, 2, true>);
            default: return ex ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 1024, 2, true, true>)
                               : go(rmsnorm_vec_kernel<TA, TW, FUSED, 1024, 2, true>);
        }
    }
    int bs = round_up((nch + kNormCPT - 1) / kNormCPT, kWave);
    // Few short rows: one chunk per lane, so the row's loads are all in
    // flight at once.
    if (n_rows < 1024) bs = bs > round_up(nch, kWave) ? bs : round_up(nch, kWave);
    if (bs > 1024) bs = round_up((nch + kNormCPT - 1) / kNormCPT, kWave);
    if (bs < kWave) bs = kWave;
    if (vec && bs <= 1024) {
        // block sizes rounded up to a power of two; one chunk per lane when
        // that covers the row, else kNormCPT
        int bp = kWave;
        while (bp < bs) bp *= 2;
        const bool one = nch <= bp;
        auto go = [&](auto kern) {
            return launch(kern, dim3(n_rows), dim3(bp), 0, stream, o, ld_out, r, ld_res, x,
                          ld_in, wt, n, eps);
        };
        // (the guarded form: at 2048 rows of 4096 the exact, unguarded
        // instantiation measured 12.9 us against 12.1)
        switch (bp) {
            case 64: return one ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 64, 1>)
                                : go(rmsnorm_vec_kernel<TA, TW, FUSED, 64, kNormCPT>);
            case 128: return one ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 128, 1>)
                                 : go(rmsnorm_vec_kernel<TA, TW, FUSED, 128, kNormCPT>);
            case 256: return one ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 256, 1>)
                                 : go(rmsnorm_vec_kernel<TA, TW, FUSED, 256, kNormCPT>);
            case 512: return one ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 512, 1>)
                                 : go(rmsnorm_vec_kernel<TA, TW, FUSED, 512, kNormCPT>);
            default: return one ? go(rmsnorm_vec_kernel<TA, TW, FUSED, 1024, 1>)
                                : go(rmsnorm_vec_kernel<TA, TW, FUSED, 1024, kNormCPT>);
        }
    }
    const int lbs = n >= 1024 ? 1024 : round_up(n, kWave);
    return launch(rmsnorm_loop_kernel<TA, TW, FUSED>, dim3(n_rows), dim3(lbs), 0, stream,
                  o, ld_out, r, ld_res, x, ld_in, wt, n, eps);
}

template <bool FUSED>
static int rmsnorm_dispatch(void* out, int ld_out, void* res, int ld_res, const void* in,
                            int ld_in, const void* w, int n_rows, int n, float eps,
                            int act_type, int weight_type, hipStream_t stream) {
    if (n_rows < 0 || n < 0) return JINF_HIP_ERR_INVALID;
    if (n_rows == 0 || n == 0) return JINF_HIP_OK;
    if (!out || !in || !w || (FUSED && !res)) return JINF_HIP_ERR_INVALID;
    if (ld_out < n || ld_in < n || (FUSED && ld_res < n)) return JINF_HIP_ERR_INVALID;
    if (FUSED && res == out) return JINF_HIP_ERR_INVALID;
    if (act_type == JINF_HIP_F32) {
        if (weight_type == JINF_HIP_F32)
            return rmsnorm_launch<float, float, FUSED>(out, ld_out, res, ld_res, in, ld_in, w,
                                                       n_rows, n, eps, stream);
        if (weight_type == JINF_HIP_F16)
            return rmsnorm_launch<float, uint16_t, FUSED>(out, ld_out, res, ld_res, in, ld_in,
                                                          w, n_rows, n, eps, stream);
    } else if (act_type == JINF_HIP_F16) {
        if (weight_type == JINF_HIP_F32)
            return rmsnorm_launch<uint16_t, float, FUSED>(out, ld_out, res, ld_res, in, ld_in,
                                                          w, n_rows, n, eps, stream);
        if (weight_type == JINF_HIP_F16)
            return rmsnorm_launch<uint16_t, uint16_t, FUSED>(out, ld_out, res, ld_res, in,
                                                             ld_in, w, n_rows, n, eps, stream);
    }
    return JINF_HIP_ERR_INVALID;
}

}  // namespace jinf

extern "C" int jinf_rmsnorm_rows(void* out, int ld_out, const void* in, int ld_in,
                                 const void* weight, int n_rows, int n, float eps,
                                 int act_type, int weight_type, hipStream_t stream) {
    return jinf::rmsnorm_dispatch<false>(out, ld_out, nullptr, 0, in, ld_in, weight, n_rows, n,
                                         eps, act_type, weight_type, stream);
}

extern "C" int jinf_residual_rmsnorm_rows(void* out, int ld_out, void* residual, int ld_res,
                                          const void* delta, int ld_delta, const void* weight,
                                          int n_rows, int n, float eps, int act_type,
                                          int weight_type, hipStream_t stream) {
    return jinf::rmsnorm_dispatch<true>(out, ld_out, residual, ld_res, delta, ld_delta, weight,
                                        n_rows, n, eps, act_type, weight_type, stream);
}

// Drop-in for the reference launcher (cuda/rmsnorm_kernel.cu:65-85): one fp32
// row; weight_type 1 = fp16 weight, every other value = fp32 weight.
extern "C" void jinf_cuda_rmsnorm(float* output, const float* input, const void* weight, int n,
                                  float eps, int weight_type, hipStream_t stream) {
    if (n <= 0) return;
    const int wt = weight_type == JINF_HIP_F16 ? JINF_HIP_F16 : JINF_HIP_F32;
    const int st = jinf::rmsnorm_dispatch<false>(output, n, nullptr, 0, input, n, weight, 1, n,
                                                 eps, JINF_HIP_F32, wt, stream);
    if (st == JINF_HIP_ERR_INVALID) JINF_LOG("jinf_cuda_rmsnorm: invalid argument (n=%d)", n);
}
