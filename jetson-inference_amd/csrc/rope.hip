// Interleaved (GGUF llama "normal") RoPE for Q and K under GQA, gfx950.
//
// Semantics (reference cuda/rope_kernel.cu:8-50), for a token at position p,
// every q head then every k head, pair i in [0, head_dim/2):
//   theta_i = fl32(base ^ (-2i / head_dim))
//   a       = fl32((float)p * theta_i)
//   c, s    = fl32(cos a), fl32(sin a)
//   x0' = x0*c - x1*s,  x1' = x0*s + x1*c   on elements (2i, 2i+1) of the head
// with every product and sum rounded to fp32 (no contraction), then one
// rounding to the storage type.
//
// Design:
//   - theta_i depends only on (base, head_dim); the host evaluates it once per
//     call in fp64 and rounds it to fp32 (the correctly rounded value), and
//     passes the table by value in the kernel arguments;
//   - grid = (units of one token / 128, tokens): a 16-byte unit is 4 (fp32)
//     or 8 (fp16) elements of one head.  Each workgroup first issues its unit
//     loads, then lanes 0..head_dim/2-1 evaluate the token's (cos, sin) pairs
//     in fp64 from the fp32 angle (full-range argument reduction), round them
//     to fp32 and share them through LDS, so the transcendental cost is paid
//     once per token per workgroup instead of once per element, and the
//     fp32 results are the correctly rounded cos/sin of the exact fp32 angle;
//   - in place: each unit is read and written by the same lane.
#include <math.h>

#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"
#include "rope_device.h"

namespace jinf {

constexpr int kRopeBlock = 128;

// Fill cs[i] = (cos, sin) of fl32(pos * theta_i) for i < half.  Ends with a
// barrier.
__device__ __forceinline__ void rope_table(float2* cs, int half, int pos,
                                           const RopeTheta& th) {
    for (int i = threadIdx.x; i < half; i += blockDim.x) cs[i] = rope_cs(pos, th.t[i]);
    __syncthreads();
}

// UPT units per thread, spaced one workgroup apart.
template <typename TA, int UPT = 1>
__global__ __launch_bounds__(kRopeBlock) void rope_vec_kernel(
    TA* q, int ld_q, TA* k, int ld_k, const int32_t* positions, int pos0, int head_dim,
    int units_q, int units_tok, RopeTheta th) {
    using A = Act<TA>;
    constexpr int E = A::kElems;
    __shared__ float2 cs[kRopeMaxHalf];
    const int64_t t = blockIdx.x;
    TA* p[UPT];
    int i0[UPT];
    uint4 raw[UPT];
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
        const int u = (blockIdx.y * UPT + j) * kRopeBlock + threadIdx.x;
        p[j] = nullptr;
        i0[j] = 0;
        if (u < units_tok) {
            const int uu = u < units_q ? u : u - units_q;
            p[j] = u < units_q ? q + t * ld_q + (int64_t)uu * E : k + t * ld_k + (int64_t)uu * E;
            i0[j] = (uu * E % head_dim) / 2;
            raw[j] = ld16<true>(p[j]);
        }
    }
    const int pos = positions ? positions[t] : pos0 + (int)t;
    rope_table(cs, head_dim / 2, pos, th);
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
        if (p[j]) {
            float v[E];
            A::unpack(raw[j], v);
#pragma unroll
            for (int e = 0; e < E / 2; ++e) {
                const float2 c = cs[i0[j] + e];
                rot(v[2 * e], v[2 * e + 1], c.x, c.y);
            }
            st16<true>(p[j], A::pack(v));
        }
    }
}

// One pair per lane, any alignment.
template <typename TA>
__global__ __launch_bounds__(kRopeBlock) void rope_scalar_kernel(
    TA* q, int ld_q, TA* k, int ld_k, const int32_t* positions, int pos0, int head_dim,
    int pairs_q, int pairs_tok, RopeTheta th) {
    using A = Act<TA>;
    __shared__ float2 cs[kRopeMaxHalf];
    const int64_t t = blockIdx.x;
    const int u = blockIdx.y * kRopeBlock + threadIdx.x;
    const int half = head_dim / 2;
    TA* p = nullptr;
    float x0 = 0.f, x1 = 0.f;
    int i = 0;
    if (u < pairs_tok) {
        const int uu = u < pairs_q ? u : u - pairs_q;
        const int head = uu / half;
        i = uu % half;
        p = (u < pairs_q ? q + t * ld_q : k + t * ld_k) + (int64_t)head * head_dim + 2 * i;
        x0 = A::load1(p);
        x1 = A::load1(p + 1);
    }
    const int pos = positions ? positions[t] : pos0 + (int)t;
    rope_table(cs, half, pos, th);
    if (u < pairs_tok) {
        const float2 c = cs[i];
        rot(x0, x1, c.x, c.y);
        A::store1(p, x0);
        A::store1(p + 1, x1);
    }
}

template <typename TA>
static int rope_launch(void* q, int ld_q, void* k, int ld_k, const int32_t* positions, int pos0,
                       int n_tokens, int head_dim, int n_heads, int n_heads_kv, float base,
                       hipStream_t stream) {
    constexpr int E = Act<TA>::kElems;
    RopeTheta th;
    theta_table(th, head_dim, base);
    TA* pq = static_cast<TA*>(q);
    TA* pk = static_cast<TA*>(k);
    const bool vec = head_dim % E == 0 && (n_heads == 0 || aligned(q, 16)) &&
                     (n_heads_kv == 0 || aligned(k, 16)) &&
                     ((int64_t)ld_q * sizeof(TA)) % 16 == 0 &&
                     ((int64_t)ld_k * sizeof(TA)) % 16 == 0;
    if (vec) {
        const int units_q = n_heads * head_dim / E;
        const int units_tok = units_q + n_heads_kv * head_dim / E;
        const dim3 grid(n_tokens, (units_tok + kRopeBlock - 1) / kRopeBlock);
        return launch(rope_vec_kernel<TA>, grid, dim3(kRopeBlock), 0, stream, pq, ld_q, pk,
                      ld_k, positions, pos0, head_dim, units_q, units_tok, th);
    }
    const int pairs_q = n_heads * head_dim / 2;
    const int pairs_tok = pairs_q + n_heads_kv * head_dim / 2;
    const dim3 grid(n_tokens, (pairs_tok + kRopeBlock - 1) / kRopeBlock);
    return launch(rope_scalar_kernel<TA>, grid, dim3(kRopeBlock), 0, stream, pq, ld_q, pk, ld_k,
                  positions, pos0, head_dim, pairs_q, pairs_tok, th);
}

static int rope_dispatch(void* q, int ld_q, void* k, int ld_k, const int32_t* positions,
                         int pos0, int n_tokens, int head_dim, int n_heads, int n_heads_kv,
                         float base, int act_type, hipStream_t stream) {
    if (n_tokens < 0 || n_heads < 0 || n_heads_kv < 0 || head_dim < 0)
        return JINF_HIP_ERR_INVALID;
    if (n_tokens == 0 || head_dim == 0 || n_heads + n_heads_kv == 0) return JINF_HIP_OK;
    if (head_dim % 2 != 0 || head_dim / 2 > kRopeMaxHalf) return JINF_HIP_ERR_INVALID;
    if ((n_heads > 0 && (!q || ld_q < n_heads * head_dim)) ||
        (n_heads_kv > 0 && (!k || ld_k < n_heads_kv * head_dim)))
        return JINF_HIP_ERR_INVALID;
    if ((int64_t)(n_heads + n_heads_kv) * head_dim / 2 > 65535LL * kRopeBlock)
        return JINF_HIP_ERR_INVALID;
    if (act_type == JINF_HIP_F32)
        return rope_launch<float>(q, ld_q, k, ld_k, positions, pos0, n_tokens, head_dim, n_heads,
                                  n_heads_kv, base, stream);
    if (act_type == JINF_HIP_F16)
        return rope_launch<uint16_t>(q, ld_q, k, ld_k, positions, pos0, n_tokens, head_dim,
                                     n_heads, n_heads_kv, base, stream);
    return JINF_HIP_ERR_INVALID;
}

}  // namespace jinf

extern "C" int jinf_rope_rows(void* q, int ld_q, void* k, int ld_k, const int32_t* positions,
                              int pos0, int n_tokens, int head_dim, int n_heads, int n_heads_kv,
                              float freq_base, int act_type, hipStream_t stream) {
    return jinf::rope_dispatch(q, ld_q, k, ld_k, positions, pos0, n_tokens, head_dim, n_heads,
                               n_heads_kv, freq_base, act_type, stream);
}

// Drop-in for cuda/rope_kernel.cu:54-61: one fp32 token at `pos`.
extern "C" void jinf_cuda_rope(float* q, float* k, int head_dim, int n_heads, int n_heads_kv,
                               int pos, float freq_base, hipStream_t stream) {
    if (head_dim <= 0 || n_heads + n_heads_kv <= 0) return;
    const int st = jinf::rope_dispatch(q, n_heads * head_dim, k, n_heads_kv * head_dim, nullptr,
                                       pos, 1, head_dim, n_heads, n_heads_kv, freq_base,
                                       JINF_HIP_F32, stream);
    if (st == JINF_HIP_ERR_INVALID)
        JINF_LOG("jinf_cuda_rope: invalid argument (head_dim=%d)", head_dim);
}
