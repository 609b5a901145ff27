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
//     or 8 (fp16) elements of one head, one unit per lane, read and written
//     by the same lane (in place) with nontemporal 16-byte accesses;
//   - head_dim <= 128 (at most 64 pairs): every wave builds the token's
//     (cos, sin) table by itself.  Lane j evaluates pair j mod head_dim/2 in
//     fp64 from the fp32 angle (cos_sin_f32: correctly rounded in practice,
//     about 25 fp64 operations) while its unit load is in flight, and each
//     lane then reads the pairs of its unit from the owning lanes with
//     cross-lane permutes.  No LDS, no barrier: a wave's stores wait only for
//     its own loads and the permutes;
//   - head_dim in (128, 512]: the workgroup's first head_dim/2 lanes build the
//     table in LDS behind one barrier.
#include <math.h>

#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"
#include "rope_device.h"

namespace jinf {

constexpr int kRopeBlock = 128;

// One 16-byte unit per lane.  WAVE_TABLE: head_dim / 2 <= 64, the (cos, sin)
// pairs come from lanes of the same wave; otherwise from an LDS table.  HD > 0
// fixes head_dim at compile time (64 and 128: the index arithmetic becomes
// shifts and masks instead of integer divisions).
template <typename TA, bool WAVE_TABLE, int HD, typename TH>
__global__ __launch_bounds__(kRopeBlock) void rope_vec_kernel(
    TA* q, int ld_q, TA* k, int ld_k, const int32_t* positions, int pos0, int head_dim_arg,
    int units_q, int units_tok, TH th) {
    using A = Act<TA>;
    constexpr int E = A::kElems;
    const int head_dim = HD > 0 ? HD : head_dim_arg;
    __shared__ float2 cs[WAVE_TABLE ? 1 : kRopeMaxHalf];
    const int64_t t = blockIdx.x;
    const int u = blockIdx.y * kRopeBlock + threadIdx.x;
    const bool live = u < units_tok;
    const int half = head_dim / 2;
    const int lane = threadIdx.x & (kWave - 1);
    // theta (a per-lane read of the kernel arguments, a vector load) is read
    // before the unit load is issued: vector loads complete in order, so a
    // later theta load would make the (cos, sin) evaluation wait for the
    // unit's HBM latency instead of overlapping it.
    float theta = 0.0f;
    if constexpr (WAVE_TABLE) theta = th.t[lane % half];
    // Lanes past the token's last unit load that unit too (never stored), so
    // every lane issues exactly one unit load and the wait for theta can
    // leave it in flight.
    const int ul = live ? u : units_tok - 1;
    const int uu = ul < units_q ? ul : ul - units_q;
    TA* p = ul < units_q ? q + t * ld_q + (int64_t)uu * E : k + t * ld_k + (int64_t)uu * E;
    const int i0 = (uu * E % head_dim) / 2;
    const uint4 raw = ld16<true>(p);
    const int pos = positions ? positions[t] : pos0 + (int)t;
    float c[E / 2], sn[E / 2];
    if constexpr (WAVE_TABLE) {
        // every lane of the wave takes part in the permutes (no lane has exited)
        const float2 mine = rope_cs(pos, theta);
#pragma unroll
        for (int e = 0; e < E / 2; ++e) {
            c[e] = __shfl(mine.x, i0 + e, kWave);
            sn[e] = __shfl(mine.y, i0 + e, kWave);
        }
    } else {
        for (int i = threadIdx.x; i < half; i += blockDim.x) cs[i] = rope_cs(pos, th.t[i]);
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E / 2; ++e) {
            c[e] = cs[i0 + e].x;
            sn[e] = cs[i0 + e].y;
        }
    }
    if (!live) return;
    float v[E];
    A::unpack(raw, v);
#pragma unroll
    for (int e = 0; e < E / 2; ++e) rot(v[2 * e], v[2 * e + 1], c[e], sn[e]);
    st16<true>(p, A::pack(v));
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
    for (int j = threadIdx.x; j < half; j += blockDim.x) cs[j] = rope_cs(pos, th.t[j]);
    __syncthreads();
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
        auto go = [&](auto kern, const auto& th) {
            return launch(kern, grid, dim3(kRopeBlock), 0, stream, pq, ld_q, pk, ld_k, positions,
                          pos0, head_dim, units_q, units_tok, th);
        };
        if (head_dim / 2 <= kWave) {
            RopeTheta64 th;
            theta_table(th, head_dim, base);
            if (head_dim == 128) return go(rope_vec_kernel<TA, true, 128, RopeTheta64>, th);
            if (head_dim == 64) return go(rope_vec_kernel<TA, true, 64, RopeTheta64>, th);
            return go(rope_vec_kernel<TA, true, 0, RopeTheta64>, th);
        }
        RopeTheta th;
        theta_table(th, head_dim, base);
        return go(rope_vec_kernel<TA, false, 0, RopeTheta>, th);
    }
    RopeTheta th;
    theta_table(th, head_dim, base);
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
