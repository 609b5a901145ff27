// GQA decode attention for gfx950: one new query token per sequence against
// its KV cache.
//
// Semantics (reference cuda/attention_kernel.cu:25-96, called from
// src/engine.cpp:446-459 after the K/V rows of the current token are written
// at position n_past): for query head h, kv head j = h / (n_heads / n_heads_kv),
//   score_t = (q_h . k_t) * scale,  t < len        (scale = 1/sqrt(head_dim))
//   out_h   = sum_t softmax(score)_t * v_t
// in fp32.  The cache of one sequence is [position][kv head][head_dim] with
// ld_pos elements between positions (n_heads_kv * head_dim in the engine);
// fp32 as in the reference, or fp16 (one rounding of the fp32 K/V rows).
//
// Design.  Decode attention streams the K and V rows once (2 * head_dim *
// bytes per position and kv head) and is HBM-bound.  A workgroup owns one
// (sequence, kv head) and the G query heads that read it, so each K/V byte is
// fetched once for the whole GQA group; its waves split the positions into
// 64-position tiles and keep flash-decoding state (running max m, sum l and
// the output accumulator) in registers.  An fp16 cache runs on the matrix
// cores (attn_mfma_kernel below); an fp32 cache (the reference's drop-in) on
// the vector ALUs:
//   - scores: LPP lanes per position, each with head_dim / LPP dims of every
//     query head in registers (LPP chosen so that G * head_dim / LPP <= 64
//     registers), load their slice of the K row (the row is read coalesced)
//     and reduce the partial dots across the LPP lanes; the score goes to LDS;
//   - softmax: lane t takes position t of the tile: one tile max and one sum
//     per head (DPP wave reductions), one exp per position and head, and the
//     probabilities go back to LDS;
//   - P V: lane l owns dims l, l + 64, ... of every head; each V row is read
//     coalesced once and multiplied into all G heads with probabilities read
//     from LDS as broadcasts;
//   - the waves' states merge through LDS at the end (flash-decoding combine,
//     in wave order).
// When there are too few (sequence, kv head) pairs to fill the GPU (batch-1
// decode), each workgroup takes a single query head instead (the G heads of
// a group then share the K/V bytes through L2) and gets up to 16 waves.
// The reference's interface has no workspace, so the positions of one head
// are not split across workgroups.
//
// head_dim 64 and 128 with 16-byte aligned rows take this kernel; anything
// else takes a one-wave-per-head kernel (dims on lanes, one wave reduction
// per position) with the same arithmetic.
#include <atomic>
#include <mutex>

#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"
#include "matvec_batch_internal.h"
#include "jinf/kernels_ext.h"

namespace jinf {

constexpr int kAtTile = 64;  // positions per tile (one per lane in the softmax step)

template <typename T> struct KV;
template <> struct KV<float> {
    static __device__ __forceinline__ float get(const float* p, int i) { return p[i]; }
};
template <> struct KV<uint16_t> {
    static __device__ __forceinline__ float get(const uint16_t* p, int i) { return h2f(p[i]); }
};

// n consecutive elements (n * sizeof(T) a multiple of 16, p 16-byte aligned)
// widened to fp32.
template <typename T, int N>
__device__ __forceinline__ void load_row(const T* p, float (&f)[N]) {
    if constexpr (sizeof(T) == 4) {
        static_assert(N % 4 == 0, "fp32 slices are whole 16-byte chunks");
#pragma unroll
        for (int c = 0; c < N / 4; ++c) {
            const float4 v = reinterpret_cast<const float4*>(p)[c];
            f[4 * c] = v.x; f[4 * c + 1] = v.y; f[4 * c + 2] = v.z; f[4 * c + 3] = v.w;
        }
    } else {
        static_assert(N % 8 == 0, "fp16 slices are whole 16-byte chunks");
#pragma unroll
        for (int c = 0; c < N / 8; ++c) {
            const uint4 v = reinterpret_cast<const uint4*>(p)[c];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[8 * c + 2 * i] = h2f((uint16_t)(w[i] & 0xFFFFu));
                f[8 * c + 2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
            }
        }
    }
}

// Sum over aligned groups of L consecutive lanes (L a power of two <= 16):
// every lane of the group gets the group's sum.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (L >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (L >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (L >= 8) v += __shfl_xor(v, 4, kWave);
    if constexpr (L >= 16) v += __shfl_xor(v, 8, kWave);
    return v;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// grid: (n_heads_kv * group / G, n_seq); block: waves * 64 (G > 1: 4 waves;
// G == 1: up to 16).
// LDS: waves * G * 64 floats (scores / probabilities), then the merge area
// waves * G * (HD + 2) floats.
template <typename TKV, int HD, int G>
__global__ __launch_bounds__(G == 1 ? 1024 : 256) void attn_decode_kernel(
    float* __restrict__ out, int64_t ld_out, const float* __restrict__ q, int64_t ld_q,
    const TKV* __restrict__ kc, const TKV* __restrict__ vc, int64_t ld_pos, int64_t ld_seq,
    const int32_t* __restrict__ lens, int n_past, int group, float scale) {
    // lens[s] is clamped to [0, n_past] (n_past = the cache's positions)
    // lanes per position: G * DPQ <= 64 q registers and a K slice of <= 32
    constexpr int LPP = (HD * G / 64) > (HD / 32) ? (HD * G / 64) : (HD / 32);
    constexpr int DPQ = HD / LPP;                                // q/k dims per lane
    constexpr int PPP = kWave / LPP;                             // positions per pass
    constexpr int NPASS = kAtTile / PPP;
    constexpr int DPL = HD / kWave;                              // P V dims per lane
    static_assert(LPP <= 16 && DPQ * G <= 64 && DPQ >= 8 && DPQ <= 32, "tile shape");
    extern __shared__ float at_lds[];
    const int waves = blockDim.x / kWave;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int s = blockIdx.y;
    const int h0 = blockIdx.x * G;      // first query head of this workgroup
    const int j = h0 / group;           // its kv head
    const int len = lens ? min(max(lens[s], 0), n_past) : n_past;
    float* sc = at_lds + wave * G * kAtTile;  // this wave's scores [G][64]

    const TKV* kb = kc + (int64_t)s * ld_seq + (int64_t)j * HD;
    const TKV* vb = vc + (int64_t)s * ld_seq + (int64_t)j * HD;
    const int sub = lane % LPP;  // which DPQ-slice of the row this lane holds

    float qv[G][DPQ];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qh = q + (int64_t)s * ld_q + (int64_t)(h0 + g) * HD + sub * DPQ;
#pragma unroll
        for (int c = 0; c < DPQ / 4; ++c) {
            const float4 v = reinterpret_cast<const float4*>(qh)[c];
            qv[g][4 * c] = v.x; qv[g][4 * c + 1] = v.y; qv[g][4 * c + 2] = v.z; qv[g][4 * c + 3] = v.w;
        }
    }

    float m[G], l[G], acc[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[g][i] = 0.0f;
    }

    for (int t0 = wave * kAtTile; t0 < len; t0 += waves * kAtTile) {
        // scores of the tile
#pragma unroll 2
        for (int pass = 0; pass < NPASS; ++pass) {
            const int pt = pass * PPP + lane / LPP;  // position within the tile
            const int pos = t0 + pt < len ? t0 + pt : len - 1;
            float kf[DPQ];
            load_row<TKV, DPQ>(kb + (int64_t)pos * ld_pos + sub * DPQ, kf);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < DPQ; ++i) d = fmaf(qv[g][i], kf[i], d);
                d = group_sum<LPP>(d);
                if (sub == 0) sc[g * kAtTile + pt] = t0 + pt < len ? d * scale : -INFINITY;
            }
        }
        wave_lds_sync();
        // online softmax over the tile: lane = position
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float st = sc[g * kAtTile + lane];
            const float mn = fmaxf(m[g], wave_max_f32(st));  // finite: position t0 is live
            const float corr = exp_neg_fast(m[g] - mn);             // 0 on the first tile
            const float p = exp_neg_fast(st - mn);
            l[g] = fmaf(l[g], corr, wave_sum_f32(p));
            m[g] = mn;
            sc[g * kAtTile + lane] = p;
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[g][i] *= corr;
        }
        wave_lds_sync();
        // P V, 8 positions at a time with their V loads issued together
        // (rows past the end re-read the last live row; their p is 0)
        const int nt = len - t0 < kAtTile ? len - t0 : kAtTile;
        const TKV* vt = vb + (int64_t)t0 * ld_pos + lane;
        for (int t = 0; t < nt; t += 8) {
            float vv[8][DPL];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int tt = t + u < nt ? t + u : nt - 1;
#pragma unroll
                for (int i = 0; i < DPL; ++i) vv[u][i] = KV<TKV>::get(vt + (int64_t)tt * ld_pos, i * kWave);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = sc[g * kAtTile + t + u];
#pragma unroll
                    for (int i = 0; i < DPL; ++i) acc[g][i] = fmaf(p, vv[u][i], acc[g][i]);
                }
        }
        wave_lds_sync();
    }

    // merge the waves' states in wave order
    float* mg = at_lds + waves * G * kAtTile;  // [waves][G][HD + 2]
    constexpr int MS = HD + 2;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float* e = mg + (wave * G + g) * MS;
#pragma unroll
        for (int i = 0; i < DPL; ++i) e[lane + i * kWave] = acc[g][i];
        if (lane == 0) {
            e[HD] = m[g];
            e[HD + 1] = l[g];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        float M = -INFINITY;
        for (int w = 0; w < waves; ++w) M = fmaxf(M, mg[(w * G + g) * MS + HD]);
        float num = 0.0f, den = 0.0f;
        for (int w = 0; w < waves; ++w) {
            const float* e = mg + (w * G + g) * MS;
            const float f = exp_neg_fast(e[HD] - M);  // idle waves: m = -inf -> 0
            num = fmaf(f, e[d], num);
            den = fmaf(f, e[HD + 1], den);
        }
        out[(int64_t)s * ld_out + (int64_t)(h0 + g) * HD + d] = len > 0 ? num / den : 0.0f;
    }
}

// Any head_dim (<= 1024) and alignment: one wave per (sequence, query head);
// lane l owns dims l, l + 64, ...; one wave reduction per position for the
// score; online softmax per position.
template <typename TKV>
__global__ __launch_bounds__(64) void attn_decode_any_kernel(
    float* __restrict__ out, int64_t ld_out, const float* __restrict__ q, int64_t ld_q,
    const TKV* __restrict__ kc, const TKV* __restrict__ vc, int64_t ld_pos, int64_t ld_seq,
    const int32_t* __restrict__ lens, int n_past, int group, int hd, float scale) {
    constexpr int kMaxDPL = 16;
    const int lane = threadIdx.x;
    const int h = blockIdx.x, s = blockIdx.y;
    const int j = h / group;
    const int len = lens ? min(max(lens[s], 0), n_past) : n_past;
    const TKV* kb = kc + (int64_t)s * ld_seq + (int64_t)j * hd;
    const TKV* vb = vc + (int64_t)s * ld_seq + (int64_t)j * hd;
    const float* qh = q + (int64_t)s * ld_q + (int64_t)h * hd;
    float qv[kMaxDPL], acc[kMaxDPL];
#pragma unroll
    for (int i = 0; i < kMaxDPL; ++i) {
        const int d = lane + i * kWave;
        qv[i] = d < hd ? qh[d] : 0.0f;
        acc[i] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    for (int t = 0; t < len; ++t) {
        const TKV* kt = kb + (int64_t)t * ld_pos;
        const TKV* vt = vb + (int64_t)t * ld_pos;
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxDPL; ++i) {
            const int d = lane + i * kWave;
            if (d < hd) part = fmaf(qv[i], KV<TKV>::get(kt, d), part);
        }
        const float st = wave_sum_f32(part) * scale;
        const float mn = fmaxf(m, st);
        const float corr = exp_neg_fast(m - mn);
        const float p = exp_neg_fast(st - mn);
        l = fmaf(l, corr, p);
        m = mn;
#pragma unroll
        for (int i = 0; i < kMaxDPL; ++i) {
            const int d = lane + i * kWave;
            if (d < hd) acc[i] = fmaf(p, KV<TKV>::get(vt, d), acc[i] * corr);
        }
    }
    float* oh = out + (int64_t)s * ld_out + (int64_t)h * hd;
#pragma unroll
    for (int i = 0; i < kMaxDPL; ++i) {
        const int d = lane + i * kWave;
        if (d < hd) oh[d] = len > 0 ? acc[i] / l : 0.0f;
    }
}

// ---- fp16 cache: matrix-core kernel ----
//
// For an fp16 cache the GQA group's work per 64-position tile is two small
// matrix products, done on the matrix cores with v_mfma_f32_16x16x32_f16
// (A 16 rows x 32 k, B 32 k x 16 columns, fp32 accumulate; lane l supplies A
// row l % 16 / B column l % 16 at eight k slots of lane group l / 16, and
// holds D rows 4 (l / 16) .. + 3 of column l % 16; the products only need the
// same k slots in A and B):
//   S^T[t][c] = sum_d K[t][d] Q'[d][c]   A = K rows (fp16, exact),
//                                          B = columns c = 8 head slots x {hi, lo}
//   O[c][d]  += sum_t P'[c][t] V[t][d]   A = P' (hi / lo rows), B = V
// q' = q * scale and P' = p * 2^15 are split into fp16 hi + lo parts
// (hi = fp16(x), lo = fp16(x - hi)), so the products keep about 22
// significant bits; the 2^15 keeps the probabilities in fp16's normal range
// and is divided out exactly at the end.  The score accumulator's layout
// (lane: column c, rows = 4 positions) is the A layout P needs, so the
// softmax runs in registers, and two 16-position blocks' accumulators make
// one 32-deep A fragment; V goes through LDS and is read back transposed.
// The dot-product index is permuted identically in K and Q' (lane group g,
// k-step s covers dims (HD/4) g + 8 s .. + 7), so each lane reads its K
// slice as whole 16-byte pieces.  (16x16x16 steps, as the one-block-per-wave
// short-context form still uses for P V, measured 234.1 against 233.0 us on
// the 70B decode attention.)
// Every exponential here (probabilities, rescale and merge factors, all of
// arguments <= 0) is the two-operation exp_neg_fast: relative error below
// 6.5e-6 for every normal result, inside the 2e-5 output bar; against a
// six-operation Cody-Waite form (about 2 ulp), the 70B decode launch
// 233.3-233.5 -> 232.0-232.1 us
// and the 8B decode step 1.363 -> 1.351 ms (interleaved on one box).
typedef _Float16 am_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 am_h8 __attribute__((ext_vector_type(8)));
typedef float am_f4 __attribute__((ext_vector_type(4)));

// A workspace splits contexts into chunks of kAmChunkMin positions or more,
// sized so that about kAmTargetItems work items fill the GPU (few, long
// sequences get short chunks; many sequences long ones).
constexpr int kAmChunkMin = 256;
constexpr int kAmTargetItems = 1024;
constexpr float kAmPScale = 32768.0f;  // 2^15
// below this many (sequence, head group) pairs a split context is merged by
// the attention kernel itself, at or above it by a second launch
constexpr int kAmInKernelMerge = 128;

__device__ __forceinline__ am_h4 am_h4_from(uint32_t lo, uint32_t hi) {
    const uint2 u = make_uint2(lo, hi);
    return __builtin_bit_cast(am_h4, u);
}
__device__ __forceinline__ am_h8 am_h8_cat(am_h4 a, am_h4 b) {
    return am_h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ float ror8(float v) { return dpp_f32<0x128>(v); }  // row_ror:8

// The in-kernel merge of a split context (attn_mfma_kernel with MERGE): the
// calling workgroup has stored its records for head slots [h0, h0 + G) of
// sequence s.  `lds` is the kernel's dynamic LDS, free at this point.
template <int HD>
__device__ __forceinline__ void am_merge_last(float* __restrict__ out, int64_t ld_out,
                                              float* __restrict__ ws,
                                              unsigned* __restrict__ counters, int s, int n_heads,
                                              int h0, int G, int nch, int used, uint8_t* lds) {
    constexpr int MS = HD + 2;
    // The last of the `used` workgroups of this (sequence, head group) merges
    // their records in chunk order and returns the counter to zero.  Records
    // are written and read with device-coherent accesses (they bypass the
    // per-XCD L2 caches, which are not coherent with one another).  Ordering:
    // every thread waits for its record stores, the barrier (a workgroup-scope
    // release / acquire) orders them before thread 0's counter update, an
    // agent-scope release increment; the workgroup that sees the final count
    // then acquires, so it synchronizes with every earlier release, and its
    // threads read the records after the barrier that follows.  Only the
    // merging workgroup pays the acquire's L2 invalidation.  (Agent-scope
    // release fences in every wave instead cost 19 -> 28 us at batch 1, 8192
    // positions: each writes back the whole L2.  A relaxed increment, relying
    // on the device-coherent accesses alone, measured the same as this on the
    // decode and 70B attention workloads.)
    __shared__ int am_last;
    __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned* cnt = counters + (int64_t)s * n_heads + blockIdx.x;
        const unsigned prev =
            __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        am_last = prev + 1 == (unsigned)used;
        if (am_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (am_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!am_last) return;
    // Merge: the chunks' (m, l) pairs and weights f_c = exp(m_c - M) go
    // through LDS (the tile buffers are free now), computed once per (chunk,
    // head) in parallel; then each (head, dim) sums f_c O_c[d] over the chunks
    // with the loads of several chunks in flight.  Same operations in the same
    // order per output as a sequential merge.
    float* mw = reinterpret_cast<float*>(lds);  // [used][8]: m, then f
    float* ml = mw + used * 8;                  // [used][8]: l
    float* mM = ml + used * 8;                  // [8]: M per head slot
    for (int idx = threadIdx.x; idx < used * G; idx += blockDim.x) {
        const int c = idx / G, g = idx % G;
        const float* e = ws + (((int64_t)s * n_heads + h0 + g) * nch + c) * MS;
        mw[c * 8 + g] = rec_load(e + HD);
        ml[c * 8 + g] = rec_load(e + HD + 1);
    }
    __syncthreads();
    if (threadIdx.x < G) {
        float M = -INFINITY;
        for (int c = 0; c < used; ++c) M = fmaxf(M, mw[c * 8 + threadIdx.x]);
        mM[threadIdx.x] = M;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < used * G; idx += blockDim.x) {
        const int c = idx / G, g = idx % G;
        const float M = mM[g];
        mw[c * 8 + g] = M > -INFINITY ? exp_neg_fast(mw[c * 8 + g] - M) : 0.0f;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        const float* rec = ws + ((int64_t)s * n_heads + h0 + g) * nch * MS + d;
        float num = 0.0f, den = 0.0f;
        if (mM[g] > -INFINITY) {
#pragma unroll 8
            for (int c = 0; c < used; ++c) {
                const float f = mw[c * 8 + g];
                num = fmaf(f, rec_load(rec + (int64_t)c * MS), num);
                den = fmaf(f, ml[c * 8 + g], den);
            }
        }
        out[(int64_t)s * ld_out + (int64_t)(h0 + g) * HD + d] = den > 0.0f ? num / den : 0.0f;
    }
}

// grid (n_heads / G, n_seq, n_chunks), 256 threads.  ws == nullptr, or a
// context that fits in one chunk: the workgroup writes the output directly;
// otherwise each (sequence, head, chunk) writes an unnormalised partial
// {O[HD], m, l} to ws, and either the last workgroup of the (sequence, head
// group) to finish merges them (counters: one per (sequence, head group),
// zero between calls) or, counters == nullptr, attn_combine_kernel does.
typedef short am_tr4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) am_tr4 am_lds_tr4;
// The parameters the prologue needs before the first K / V loads lead the
// list: the first 14 dwords arrive preloaded in SGPRs, so those loads wait
// for one scalar round trip (the sequence's length), not for several.  (q's
// loads, which need later arguments, stay in flight behind K's.)
template <int HD, bool MERGE, bool RB>
__global__ __launch_bounds__(256) void attn_mfma_kernel(
    const int32_t* __restrict__ lens, int n_past, int chunk, int G, int group,
    const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t ld_pos,
    int64_t ld_seq, const float* __restrict__ q, int64_t ld_q, int n_heads, float scale,
    float* __restrict__ out, int64_t ld_out, float* __restrict__ ws,
    unsigned* __restrict__ counters, uint8_t* __restrict__ xrec, int xmt) {
    constexpr int KS = HD / 16;        // k-steps of the score product
    constexpr int DPG = HD / 4;        // dims per lane group in the score product
    constexpr int KLD = DPG / 8;       // 16-byte K loads per position block
    constexpr int NB = HD / 16;        // 16-dim blocks of the output
    constexpr int VCH = HD / 8;        // 16-byte chunks per V row
    constexpr int VRS = kWave / VCH;   // V rows per load instruction
    constexpr int VLD = kAtTile / VRS; // V loads per lane per tile
    // RB (short contexts): every wave walks every tile but owns one 16-row
    // block of it (block b = wave), loading only those rows: VLDW loads each
    // for K and V.  Otherwise a wave owns whole tiles (tile = 64 w + 256 k).
    constexpr int VLDW = RB ? 16 / VRS : VLD;
    constexpr int NBK = RB ? 1 : 4;    // 16-row blocks of a tile this wave processes
    constexpr int PITCH = HD * 2;      // LDS bytes per staged V row
    constexpr int MS = HD + 2;         // merge record: O[HD], m, l
    // 16-byte aligned: the merge's static LDS word comes first, and the
    // tiles' 8- and 16-byte reads need aligned addresses
    extern __shared__ __attribute__((aligned(16))) uint8_t am_lds[];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, lg = lane >> 4;
    const int slot = col & 7;          // head slot of this column
    const bool lo_col = col >= 8;
    // grid (head groups, sequences, chunks): the chunk index is the slowest
    // dimension, so every sequence's first chunk (the longest work items)
    // is dispatched before any second chunk, and the shorter or empty later
    // chunks fill the tail (64 sequences x 8192 positions: 260 -> 236 us)
    const int s = blockIdx.y;
    const int cix = blockIdx.z;
    const int h0 = blockIdx.x * G;
    // The sequence's length is the one load ahead of the K / V loads (their
    // bounds need it); every argument they need arrives preloaded.
    const int j = h0 / group;
    const int len = lens ? min(max(lens[s], 0), n_past) : n_past;
    const int c0 = cix * chunk;
    const int c1 = min(c0 + chunk, len);
    // chunks past the context have nothing to do (chunk 0 always runs, so an
    // empty context still writes its zeros)
    if (cix > 0 && c0 >= len) return;
    const int used = (len + chunk - 1) / chunk;  // chunks holding positions
    uint8_t* vst = am_lds + wave * 2 * kAtTile * PITCH;  // V tile, then K tile
    const uint16_t* kb = kc + (int64_t)s * ld_seq + (int64_t)j * HD;
    const uint16_t* vb = vc + (int64_t)s * ld_seq + (int64_t)j * HD;


    float m = -INFINITY, lsum = 0.0f;
    am_f4 O[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) O[n] = am_f4{0.f, 0.f, 0.f, 0.f};

    // Software pipeline over the wave's tiles, all loads straight to LDS
    // (global_load_lds_dwordx4: instruction i of a tile fills the wave's
    // 16-byte slots 64 i + lane, so the source address picks the layout):
    // the next tile's K rows are requested right after the current score
    // product has read the K buffer, its V rows right after the current P V
    // has read the V buffer; the waits below let the other buffer's loads
    // stay in flight.  Rows past the end read as zeros (masked out).  K slot
    // (row r, p) holds chunk p ^ swizzle(r) so that the
    // 16 rows of a fragment read hit distinct banks; V slot (r, p) holds
    // chunk p ^ 2 (r & 3), so that the four rows a 16-lane transposing read
    // touches sit in distinct bank groups.
    uint8_t* kst = vst + kAtTile * PITCH;  // this wave's K tile, after its V tile
    auto kswz = [](int r) { return HD == 128 ? (r & 15) : ((r >> 1) & 7); };
    const int i0 = RB ? VLDW * wave : 0;  // first load instruction of the wave's rows
    // Positions c0 .. c1 - 1 of this (sequence, kv head) as buffer resources
    // (the host keeps their bytes below 2^31).  A lane's chunk of a tile sits
    // at the same offset from the tile's first row in every tile, so those
    // offsets are computed once here and a tile adds only its wave-uniform
    // start; rows at or past c1 fall outside the resource and read as zeros
    // (their scores are masked and their probabilities are 0).
    const uint32_t rowb = (uint32_t)ld_pos * 2;
    const int nrec = (int)((uint32_t)(c1 - c0) * rowb);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(kb + (int64_t)c0 * ld_pos), (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(vb + (int64_t)c0 * ld_pos), (short)0, nrec, 0x00020000);
    uint32_t koff[VLDW], voff[VLDW];
#pragma unroll
    for (int ii = 0; ii < VLDW; ++ii) {
        const int slot_i = kWave * (i0 + ii) + lane;
        const int row = slot_i / VCH;
        koff[ii] = (uint32_t)row * rowb + 16u * (uint32_t)((slot_i % VCH) ^ kswz(row));
        voff[ii] = (uint32_t)row * rowb + 16u * (uint32_t)((slot_i % VCH) ^ (2 * (row & 3)));
    }
    // (first: nothing has read the buffers yet, so no wait; that wait would
    // also take in the scalar loads of later kernel arguments)
    auto load_k = [&](int t0, bool first = false) {
        if (!first) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only: K buffer reads are done
        const uint32_t so = (uint32_t)(t0 - c0) * rowb;
#pragma unroll
        for (int ii = 0; ii < VLDW; ++ii) lds_load16_buf(krs, koff[ii], so, kst + 1024 * (i0 + ii));
    };
    auto load_v = [&](int t0, bool first = false) {
        if (!first) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only: V buffer reads are done
        const uint32_t so = (uint32_t)(t0 - c0) * rowb;
#pragma unroll
        for (int ii = 0; ii < VLDW; ++ii) lds_load16_buf(vrs, voff[ii], so, vst + 1024 * (i0 + ii));
    };
    // the wave's first tile and step; wrow: the wave's first row in a tile
    const int tstep = RB ? kAtTile : 4 * kAtTile;
    const int tfirst = RB ? c0 : c0 + wave * kAtTile;
    const int wrow = RB ? 16 * wave : 0;
    if (tfirst + wrow < c1) {
        load_k(tfirst, true);
        load_v(tfirst, true);
    }
    // Q' fragments of this lane's column (zero for unused head slots): the
    // lane's DPG contiguous q values, loaded unconditionally after the first
    // tile's K / V loads (q's arguments are not among the preloaded ones, and
    // its loads stay in flight behind K's) and converted below.
    float4 qraw[KS];
    {
        const float4* qp = reinterpret_cast<const float4*>(
            q + (int64_t)s * ld_q + (int64_t)(h0 + (slot < G ? slot : 0)) * HD + DPG * lg);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qraw[ks] = qp[ks];
    }
    // q' = q * scale as fp16 hi / lo parts (the compiler's wait for the q
    // loads also covers the K / V loads issued after them: in-order counts)
    am_h4 qf[KS];
    {
        const float qs = slot < G ? scale : 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const float4 v = qraw[ks];
            const float x[4] = {v.x * qs, v.y * qs, v.z * qs, v.w * qs};
            _Float16 hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const _Float16 hi = (_Float16)x[i];
                hv[i] = lo_col ? (_Float16)(x[i] - (float)hi) : hi;
            }
            qf[ks] = am_h4{hv[0], hv[1], hv[2], hv[3]};
        }
    }
    // the score product's B fragments for 32-deep k-steps: the lane's 8 dims
    // DPG lg + 8 u .. + 7, the order of the K row's 16-byte chunk u
    am_h8 qf8[KLD];
#pragma unroll
    for (int u = 0; u < KLD; ++u) qf8[u] = am_h8_cat(qf[2 * u], qf[2 * u + 1]);
    // A wave stops at the first tile holding none of its rows (with RB a
    // wave's block can end before the tile does), so it never issues loads
    // for a tile it does not process and never sees an all-masked tile.
    for (int t0 = tfirst; t0 + wrow < c1; t0 += tstep) {
        const bool more = t0 + tstep + wrow < c1;  // wave-uniform
        // K(t) has landed once at most the VLDW V loads issued after it remain
        __builtin_amdgcn_s_waitcnt(waitcnt_vm<VLDW>());
        wave_lds_sync();
        // scores: A fragment = 4 halves of row 16 b + col at dims DPG lg + 4 ks
        am_f4 S[NBK];
#pragma unroll
        for (int bi = 0; bi < NBK; ++bi) {
            const int b = RB ? wave : bi;  // the block's rows in the tile: 16 b ..
            S[bi] = am_f4{0.f, 0.f, 0.f, 0.f};
            const int r = 16 * b + col;
#pragma unroll
            for (int u = 0; u < KLD; ++u) {
                const int c = (DPG * lg) / 8 + u;  // 16-byte chunk of the row
                const uint4 w = *reinterpret_cast<const uint4*>(kst + r * PITCH + 16 * (c ^ kswz(r)));
                S[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(am_h8, w), qf8[u], S[bi], 0, 0, 0);
            }
        }
        wave_lds_sync();
        if (more) load_k(t0 + tstep);
        // hi + lo columns, mask, tile max (lanes of one column: xor 16, 32)
        float tmax = -INFINITY;
#pragma unroll
        for (int bi = 0; bi < NBK; ++bi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int b = RB ? wave : bi;
                const float v = S[bi][r] + ror8(S[bi][r]);
                const float vm = t0 + 16 * b + 4 * lg + r < c1 ? v : -INFINITY;
                S[bi][r] = vm;
                tmax = fmaxf(tmax, vm);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
        tmax = xor32_max(tmax);
        const float mn = fmaxf(m, tmax);
        const float corr = exp_neg_fast(m - mn);
        m = mn;
        float psum = 0.0f;
        am_h4 P[NBK];
#pragma unroll
        for (int bi = 0; bi < NBK; ++bi) {
            _Float16 hv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pr = exp_neg_fast(S[bi][r] - mn);
                psum += pr;
                const float ps = pr * kAmPScale;
                const _Float16 hi = (_Float16)ps;
                hv[r] = lo_col ? (_Float16)(ps - (float)hi) : hi;
            }
            P[bi] = am_h4{hv[0], hv[1], hv[2], hv[3]};
        }
        lsum = fmaf(lsum, corr, psum);
        // rescale O: its rows 4 lg + r are slots (4 lg + r) & 7, whose factor
        // sits in lane slot (lane group 0)
        float cr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float c_lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr), r));
            const float c_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr), 4 + r));
            cr[r] = (lg & 1) ? c_hi : c_lo;
        }
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) O[n][r] *= cr[r];
        // O += P' V once the tile's V has landed in LDS (the next tile's K
        // loads, issued later, may stay in flight)
        if (more)
            __builtin_amdgcn_s_waitcnt(waitcnt_vm<VLDW>());
        else
            __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
        wave_lds_sync();
        // B fragment V[16 b + 4 lg + i][16 n + col], i = 0..3, through one
        // transposing LDS read (ds_read_b64_tr_b16: within each 16 lanes,
        // lane c receives element c % 4 of the 8 bytes read by lanes
        // c / 4 + 4 i): lane c reads row 16 b + 4 lg + c / 4, columns
        // 16 n + 4 (c % 4) .. + 3
        auto vfrag = [&](int b, int n) {
            const int vr = 16 * b + 4 * lg + (col >> 2);
            const uint8_t* vrow = vst + vr * PITCH + 8 * (col & 1);
            const int p = (2 * n + ((col & 3) >> 1)) ^ (2 * (vr & 3));  // swizzled chunk
            return __builtin_bit_cast(am_h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                 (am_lds_tr4*)(vrow + 16 * p)));
        };
        if constexpr (RB) {
#pragma unroll
            for (int n = 0; n < NB; ++n)
                O[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(P[0], vfrag(wave, n), O[n], 0, 0, 0);
        } else {
            // two 16-row blocks per 32-deep k-step: lane group lg's 8 k
            // slots are positions 16 b + 4 lg + i of blocks b = 2 bp and
            // 2 bp + 1, in P' (the score accumulators) and in V alike
#pragma unroll
            for (int bp = 0; bp < NBK / 2; ++bp) {
                const am_h8 pa = am_h8_cat(P[2 * bp], P[2 * bp + 1]);
#pragma unroll
                for (int n = 0; n < NB; ++n)
                    O[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        pa, am_h8_cat(vfrag(2 * bp, n), vfrag(2 * bp + 1, n)), O[n], 0, 0, 0);
            }
        }
        wave_lds_sync();
        if (more) load_v(t0 + tstep);
    }

    // hi + lo rows (lane groups 2, 3 hold the lo rows of groups 0, 1), the
    // column's probability sum over its four lane groups
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[n][r] = xor32_sum(O[n][r]);
    lsum += __shfl_xor(lsum, 16, kWave);
    lsum = xor32_sum(lsum);

    // merge the four waves (wave order) through LDS
    __syncthreads();
    float* mg = reinterpret_cast<float*>(am_lds);  // [4][8][MS]
    if (lg < 2) {
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                mg[(wave * 8 + 4 * lg + r) * MS + 16 * n + col] = O[n][r] * (1.0f / kAmPScale);
    }
    if (lg == 0 && col < 8) {
        mg[(wave * 8 + col) * MS + HD] = m;
        mg[(wave * 8 + col) * MS + HD + 1] = lsum;
    }
    __syncthreads();
    const int nch = gridDim.z;
    const bool direct = !ws || used <= 1;  // this workgroup holds the whole context
    float* ov = reinterpret_cast<float*>(am_lds + (4 * 8 * MS * 4 + 15) / 16 * 16);  // [G HD]
    float omax = 0.0f;  // largest |output| of this thread (x records)
    for (int idx = threadIdx.x; idx < G * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        float M = -INFINITY;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, mg[(w * 8 + g) * MS + HD]);
        float num = 0.0f, den = 0.0f;
        if (M > -INFINITY) {
            for (int w = 0; w < 4; ++w) {
                const float* e = mg + (w * 8 + g) * MS;
                const float f = exp_neg_fast(e[HD] - M);
                num = fmaf(f, e[d], num);
                den = fmaf(f, e[HD + 1], den);
            }
        }
        if (direct) {
            const float o = den > 0.0f ? num / den : 0.0f;
            out[(int64_t)s * ld_out + (int64_t)(h0 + g) * HD + d] = o;
            if (xrec) {
                ov[idx] = o;
                omax = fmaxf(omax, fabsf(o));
            }
        } else {
            // device-coherent stores only for the in-kernel merge; the
            // merge launch reads ordinary stores after the kernel boundary
            float* rec = ws + (((int64_t)s * n_heads + h0 + g) * nch + cix) * MS;
            if constexpr (MERGE) {
                rec_store(rec + d, num);
                if (d == 0) {
                    rec_store(rec + HD, M);
                    rec_store(rec + HD + 1, den);
                }
            } else {
                rec[d] = num;
                if (d == 0) {
                    rec[HD] = M;
                    rec[HD + 1] = den;
                }
            }
        }
    }
    if (xrec && direct) {
        // The output projection's prepared x for this workgroup's G HD
        // columns of token s (one column chunk of that GEMV's splits): the
        // power-of-two scale of their largest magnitude, then the same
        // fragments and slab data as the GEMV's own preparation writes.
        float* red = ov + G * HD;
        float mm = wave_max_f32(omax);
        if (lane == 0) red[wave] = mm;
        __syncthreads();  // ov and the wave maxima
        mm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const int ex = mb_scale_exp(mm);
        const float sc = ldexpf(1.0f, 15 - ex);
        const int t = threadIdx.x;
        const int col0 = h0 * HD + 8 * t;  // the group's first column
        const bool here = t < G * HD / 8;
        uint8_t* r = xrec + (int64_t)(col0 / 256) * mb_rec_bytes(xmt);
        const int gi = (col0 % 256) / 8;
        float sum = 0.0f;
        if (here) {
            float v8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v8[e] = ov[8 * t + e];
            sum = mb_put_group(r, s, gi, v8, sc);
        }
        // Q4_K sub-block sums: lanes 4 q .. 4 q + 3 hold one 32-column sub-block
        sum += __shfl_xor(sum, 1, kWave);
        sum += __shfl_xor(sum, 2, kWave);
        if (here) mb_put_meta(r, xmt, s, gi, sum, ex);
    }
    // Without MERGE, attn_combine_kernel merges the records.  (The merge is a
    // separate instantiation: its code in the same kernel, even unexecuted,
    // slowed the main loop by 6% at 64 sequences x 8192 positions.)
    if constexpr (MERGE) {
        if (!direct)
            am_merge_last<HD>(out, ld_out, ws, counters, s, n_heads, h0, G, nch, used, am_lds);
    } else {
        (void)counters;
    }
}

// Merge of the chunk partials in a separate launch: grid (n_heads, n_seq),
// head_dim threads; sequences whose context fits in one chunk were written
// directly by the attention kernel.
__global__ __launch_bounds__(256) void attn_combine_kernel(
    float* __restrict__ out, int64_t ld_out, const float* __restrict__ ws,
    const int32_t* __restrict__ lens, int n_past, int n_heads, int hd, int nch, int chunk) {
    const int h = blockIdx.x, s = blockIdx.y, d = threadIdx.x;
    if (d >= hd) return;
    const int len = lens ? min(max(lens[s], 0), n_past) : n_past;
    const int used = (len + chunk - 1) / chunk;
    if (used <= 1) return;
    const float* rec = ws + ((int64_t)s * n_heads + h) * nch * (hd + 2);
    float M = -INFINITY;
    for (int c = 0; c < used; ++c) M = fmaxf(M, rec[c * (hd + 2) + hd]);
    float num = 0.0f, den = 0.0f;
    if (M > -INFINITY) {
        for (int c = 0; c < used; ++c) {
            const float* e = rec + c * (hd + 2);
            const float f = exp_neg_fast(e[hd] - M);
            num = fmaf(f, e[d], num);
            den = fmaf(f, e[hd + 1], den);
        }
    }
    out[(int64_t)s * ld_out + (int64_t)h * hd + d] = den > 0.0f ? num / den : 0.0f;
}

// Workspace: one merge counter per (sequence, head group) -- n_seq * n_heads
// slots cover any grouping -- padded to 256 bytes, then the chunk records
// {O[HD], m, l} of every (sequence, head, chunk).
static size_t am_counter_bytes(int n_seq, int n_heads) {
    return ((size_t)n_seq * n_heads * sizeof(unsigned) + 255) / 256 * 256;
}

static size_t am_workspace_bytes(int n_seq, int n_heads, int head_dim, int max_ctx) {
    const int64_t nch = ((int64_t)max_ctx + kAmChunkMin - 1) / kAmChunkMin;
    return am_counter_bytes(n_seq, n_heads) +
           (size_t)n_seq * n_heads * nch * (head_dim + 2) * sizeof(float);
}

// Where a split context keeps its merge counters and chunk records.
//   fixed == false: the caller's workspace (`base`, `bytes`), laid out as
//     above and used only when it holds am_workspace_bytes for the call;
//   fixed == true: this device's copy of `scratch` (below), with a fixed
//     layout: kScratchCounterBytes of merge counters, then
//     kScratchRecordBytes of records.  A call whose split needs more runs
//     unsplit.
struct AmScratch {
    void* base;
    size_t bytes;
    bool fixed;
};

// The no-allocation entry point's scratch (jinf_attention_decode_noalloc):
// 4096 merge counters and 8 MiB of chunk records, enough for every split of
// up to about 1000 (sequence, head group) pairs at head_dim 128 (the 70B
// 64-sequence decode needs 4.3 MB).  Each device that runs the library holds
// its own copy until the process ends; host code only ever passes the
// per-device address from hipGetSymbolAddress (scratch_base), never the
// symbol itself.
constexpr size_t kScratchCounterBytes = (size_t)16 << 10;
constexpr size_t kScratchRecordBytes = (size_t)8 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchCounterBytes + kScratchRecordBytes];

// Zero n merge counters (a kernel rather than a memset node, so that the
// call stays correct when a caller captures it in a graph).
__global__ __launch_bounds__(256) void am_clear_kernel(unsigned* __restrict__ c, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) c[i] = 0u;
}

template <int HD>
static int am_launch(float* out, int64_t ld_out, const float* q, int64_t ld_q, const void* k,
                     const void* v, int64_t ld_pos, int64_t ld_seq, const int32_t* lens,
                     int n_past, int n_seq, int n_heads, int group, int G, float scale,
                     const AmScratch& sc, MbXRec* xr, hipStream_t stream) {
    const size_t shmem = (size_t)4 * 2 * kAtTile * HD * 2;  // K and V tile per wave
    // chunk: a multiple of 64 positions, at least kAmChunkMin, giving about
    // kAmTargetItems (sequence, head group, chunk) items
    const int64_t work = (int64_t)n_past * n_seq * (n_heads / G);
    int64_t ch = (work + kAmTargetItems - 1) / kAmTargetItems;
    ch = (ch + 63) / 64 * 64;
    if (ch < kAmChunkMin) ch = kAmChunkMin;
    // the merge keeps 16 floats per chunk (+ 8) in the tile buffers' LDS
    bool split = sc.base && n_past > ch &&
                 ((n_past + ch - 1) / ch * 16 + 8) * sizeof(float) <= shmem;
    if (split && !sc.fixed && sc.bytes < am_workspace_bytes(n_seq, n_heads, HD, n_past))
        split = false;
    // The fixed scratch: a split whose records or in-launch merge counters do
    // not fit runs unsplit, as a call with too small a workspace does (such a
    // split has about as many (sequence, head group) pairs as work items to
    // aim for, so the unsplit launch still fills the GPU).
    if (split && sc.fixed) {
        const size_t need = (size_t)n_seq * n_heads * ((n_past + ch - 1) / ch) * (HD + 2) *
                            sizeof(float);
        const bool ink = (int64_t)n_seq * (n_heads / G) < kAmInKernelMerge;
        if (need > kScratchRecordBytes ||
            (ink && (size_t)n_seq * n_heads * sizeof(unsigned) > kScratchCounterBytes))
            split = false;
    }
    const int chunk = split ? (int)ch : (n_past > 0 ? n_past : 1);
    const int nch = split ? (n_past + chunk - 1) / chunk : 1;
    // Few (sequence, head group) pairs: the last workgroup of each merges in
    // the same launch (measured at batch 1, 8192 positions: 19 us against 27
    // with a second launch).  Many: every chunk workgroup would wait on the
    // merge counter before retiring, so a separate wide merge launch is
    // faster (64 sequences x 8 groups: 268 us against 290).
    const bool in_kernel = (int64_t)n_seq * (n_heads / G) < kAmInKernelMerge;
    unsigned* counters = nullptr;
    float* ws = nullptr;
    if (split && sc.fixed) {
        const size_t slots = (size_t)n_seq * n_heads;  // fits: checked above
        counters = in_kernel ? static_cast<unsigned*>(sc.base) : nullptr;
        ws = reinterpret_cast<float*>(static_cast<uint8_t*>(sc.base) + kScratchCounterBytes);
        if (counters) {
            // the scratch keeps the previous call's contents: clear the counters
            const int st = launch(am_clear_kernel, dim3((unsigned)((slots + 255) / 256)),
                                  dim3(256), 0, stream, counters, (int)slots);
            if (st != JINF_HIP_OK) return st;
        }
    } else if (split) {
        counters = in_kernel ? static_cast<unsigned*>(sc.base) : nullptr;
        ws = reinterpret_cast<float*>(static_cast<char*>(sc.base) +
                                      am_counter_bytes(n_seq, n_heads));
    }
    // up to 128 positions per work item the four waves share each tile by
    // 16-row blocks (otherwise at most two waves would hold a tile)
    const bool rb = chunk <= 2 * kAtTile;
    auto* kern = counters ? (rb ? attn_mfma_kernel<HD, true, true> : attn_mfma_kernel<HD, true, false>)
                          : (rb ? attn_mfma_kernel<HD, false, true> : attn_mfma_kernel<HD, false, false>);
    // the output projection's x records, when every work item writes its
    // output directly and one item's G HD columns are one of that GEMV's
    // per-split chunks
    uint8_t* xrec = nullptr;
    if (xr && xr->rec && !split && xr->chunk_cols == G * HD && (xr->mt == 1 || xr->mt == 2) &&
        n_seq <= 32 * xr->mt)
        xrec = xr->rec;
    const int st = launch(kern, dim3(n_heads / G, n_seq, nch), dim3(256), shmem, stream, lens,
                          n_past, chunk, G, group, static_cast<const uint16_t*>(k),
                          static_cast<const uint16_t*>(v), ld_pos, ld_seq, q, ld_q, n_heads,
                          scale, out, ld_out, ws, counters, xrec, xr ? xr->mt : 1);
    if (xr) xr->wrote = st == JINF_HIP_OK && xrec != nullptr;
    if (st != JINF_HIP_OK || !split || in_kernel) return st;
    return launch(attn_combine_kernel, dim3(n_heads, n_seq), dim3(HD), 0, stream, out, ld_out,
                  (const float*)ws, lens, n_past, n_heads, HD, nch, chunk);
}

template <typename TKV, int HD, int G>
static int at_launch(float* out, int64_t ld_out, const float* q, int64_t ld_q, const void* k,
                     const void* v, int64_t ld_pos, int64_t ld_seq, const int32_t* lens,
                     int n_past, int n_seq, int n_heads, int group, int waves, float scale,
                     hipStream_t stream) {
    const size_t shmem = ((size_t)waves * G * kAtTile + (size_t)waves * G * (HD + 2)) * 4;
    return launch(attn_decode_kernel<TKV, HD, G>, dim3(n_heads / G, n_seq), dim3(waves * kWave),
                  shmem, stream, out, ld_out, q, ld_q, static_cast<const TKV*>(k),
                  static_cast<const TKV*>(v), ld_pos, ld_seq, lens, n_past, group, scale);
}

template <typename TKV, int HD>
static int at_pick_g(int G, float* out, int64_t ld_out, const float* q, int64_t ld_q,
                     const void* k, const void* v, int64_t ld_pos, int64_t ld_seq,
                     const int32_t* lens, int n_past, int n_seq, int n_heads, int group,
                     int waves, float scale, hipStream_t stream) {
    switch (G) {
        case 8: return at_launch<TKV, HD, 8>(out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq, n_heads, group, waves, scale, stream);
        case 4: return at_launch<TKV, HD, 4>(out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq, n_heads, group, waves, scale, stream);
        case 2: return at_launch<TKV, HD, 2>(out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq, n_heads, group, waves, scale, stream);
        default: return at_launch<TKV, HD, 1>(out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq, n_heads, group, waves, scale, stream);
    }
}

// Every sequence has n_past positions (the drop-in: lens == nullptr), or
// lens[s] of at most n_past (the cache's capacity) positions.
static int attention_decode(float* out, int64_t ld_out, const float* q, int64_t ld_q,
                            const void* k, const void* v, int kv_type, int64_t ld_pos,
                            int64_t ld_seq, const int32_t* lens, int n_past, int n_seq,
                            int head_dim, int n_heads, int n_heads_kv, float scale,
                            const AmScratch& sc, hipStream_t stream, MbXRec* xr = nullptr) {
    if (xr) xr->wrote = false;
    if (n_seq < 0 || head_dim <= 0 || n_heads <= 0 || n_heads_kv <= 0) return JINF_HIP_ERR_INVALID;
    if (n_seq == 0) return JINF_HIP_OK;
    if (!out || !q || !k || !v || n_heads % n_heads_kv != 0) return JINF_HIP_ERR_INVALID;
    if (kv_type != JINF_HIP_F32 && kv_type != JINF_HIP_F16) return JINF_HIP_ERR_INVALID;
    if (head_dim > 1024 || ld_pos < (int64_t)n_heads_kv * head_dim) return JINF_HIP_ERR_INVALID;
    if (ld_out < (int64_t)n_heads * head_dim || ld_q < (int64_t)n_heads * head_dim)
        return JINF_HIP_ERR_INVALID;
    if (n_seq > 65535 || n_heads > 0x7FFFFFFF / 2) return JINF_HIP_ERR_INVALID;
    if (!(scale > 0.0f) || !(scale < INFINITY)) return JINF_HIP_ERR_INVALID;
    if (!aligned(out, 4) || !aligned(q, 4)) return JINF_HIP_ERR_INVALID;
    const int group = n_heads / n_heads_kv;
    const int64_t es = kv_type == JINF_HIP_F16 ? 2 : 4;
    // (the matrix-core kernel addresses one (sequence, kv head)'s positions
    // through 32-bit buffer offsets: their bytes stay below 2^31)
    const bool fast = (head_dim == 64 || head_dim == 128) && aligned(k, 16) && aligned(v, 16) &&
                      aligned(q, 16) && (ld_pos * es) % 16 == 0 && (ld_seq * es) % 16 == 0 &&
                      ld_q % 4 == 0 &&
                      (kv_type != JINF_HIP_F16 || (int64_t)n_past * ld_pos * es <= 0x7FFFFFFF);
    if (!fast) {
        const dim3 grid(n_heads, n_seq);
        if (kv_type == JINF_HIP_F16)
            return launch(attn_decode_any_kernel<uint16_t>, grid, dim3(kWave), 0, stream, out,
                          ld_out, q, ld_q, static_cast<const uint16_t*>(k),
                          static_cast<const uint16_t*>(v), ld_pos, ld_seq, lens, n_past, group,
                          head_dim, scale);
        return launch(attn_decode_any_kernel<float>, grid, dim3(kWave), 0, stream, out, ld_out,
                      q, ld_q, static_cast<const float*>(k), static_cast<const float*>(v), ld_pos,
                      ld_seq, lens, n_past, group, head_dim, scale);
    }
    // fp16 cache: the matrix-core kernel, all query heads of a group (up to
    // 8) per workgroup.
    if (kv_type == JINF_HIP_F16) {
        const int G = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
        if (head_dim == 64)
            return am_launch<64>(out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq,
                                 n_heads, group, G, scale, sc, xr, stream);
        return am_launch<128>(out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq,
                              n_heads, group, G, scale, sc, xr, stream);
    }
    // fp32 cache: enough (sequence, kv head) pairs: one workgroup per pair,
    // all its query heads (up to 8) together.  Otherwise one query head per
    // workgroup, with more waves when the (known) context is long.
    int G = 1, waves = 4;  // G > 1 always runs 4 waves (its launch bound)
    if ((int64_t)n_seq * n_heads_kv >= 128) {
        G = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    } else {
        const int tiles = lens ? 64 : (n_past + kAtTile - 1) / kAtTile;
        waves = tiles < 4 ? 4 : tiles > 16 ? 16 : tiles;
    }
    if (head_dim == 64)
        return at_pick_g<float, 64>(G, out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq, n_heads, group, waves, scale, stream);
    return at_pick_g<float, 128>(G, out, ld_out, q, ld_q, k, v, ld_pos, ld_seq, lens, n_past, n_seq, n_heads, group, waves, scale, stream);
}

// 1/sqrt(head_dim) rounded once from fp64 (the reference uses rsqrtf).
static float inv_sqrt_hd(int head_dim) { return (float)(1.0 / sqrt((double)head_dim)); }

}  // namespace jinf

extern "C" size_t jinf_attention_workspace_bytes(int n_seq, int n_heads, int head_dim,
                                                int max_ctx) {
    if (n_seq <= 0 || n_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
    return jinf::am_workspace_bytes(n_seq, n_heads, head_dim, max_ctx);
}

extern "C" int jinf_attention_decode(float* out, int ld_out, const float* q, int ld_q,
                                     const void* k_cache, const void* v_cache, int kv_type,
                                     int64_t ld_pos, int64_t ld_seq, const int32_t* lens,
                                     int n_seq, int max_ctx, int head_dim, int n_heads,
                                     int n_heads_kv, float scale, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
    if ((!lens && n_seq > 0) || max_ctx < 0) return JINF_HIP_ERR_INVALID;
    // ld_seq 0: every sequence reads the same cache (the tokens of one prompt)
    if (n_seq > 1 && ld_seq != 0 && ld_seq < (int64_t)max_ctx * ld_pos) return JINF_HIP_ERR_INVALID;
    if (workspace && !jinf::aligned(workspace, 4)) return JINF_HIP_ERR_INVALID;
    if (scale == 0.0f && head_dim > 0) scale = jinf::inv_sqrt_hd(head_dim);
    return jinf::attention_decode(out, ld_out, q, ld_q, k_cache, v_cache, kv_type, ld_pos, ld_seq,
                                  lens, max_ctx, n_seq, head_dim, n_heads, n_heads_kv, scale,
                                  jinf::AmScratch{workspace, workspace_bytes, false}, stream);
}

namespace jinf {

int attention_decode_xrec(float* out, int ld_out, const float* q, int ld_q, const void* k_cache,
                          const void* v_cache, int kv_type, int64_t ld_pos, int64_t ld_seq,
                          const int32_t* lens, int n_seq, int max_ctx, int head_dim, int n_heads,
                          int n_heads_kv, float scale, void* workspace, size_t workspace_bytes,
                          MbXRec* xr, hipStream_t stream) {
    if (xr) xr->wrote = false;
    if ((!lens && n_seq > 0) || max_ctx < 0) return JINF_HIP_ERR_INVALID;
    if (n_seq > 1 && ld_seq != 0 && ld_seq < (int64_t)max_ctx * ld_pos) return JINF_HIP_ERR_INVALID;
    if (workspace && !aligned(workspace, 4)) return JINF_HIP_ERR_INVALID;
    if (scale == 0.0f && head_dim > 0) scale = inv_sqrt_hd(head_dim);
    return attention_decode(out, ld_out, q, ld_q, k_cache, v_cache, kv_type, ld_pos, ld_seq, lens,
                            max_ctx, n_seq, head_dim, n_heads, n_heads_kv, scale,
                            AmScratch{workspace, workspace_bytes, false}, stream, xr);
}

// This device's address of `scratch`: looked up with hipGetSymbolAddress on
// the first call made while the device is current, then cached per device.
constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_base[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_base(void** base) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        JINF_LOG("jinf_attention_decode_noalloc: no usable current device (%d)", dev);
        return JINF_HIP_ERR_DEVICE;
    }
    void* p = g_scratch_base[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_base[dev].load(std::memory_order_relaxed);
        if (!p) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                JINF_LOG("jinf_attention_decode_noalloc: hipGetSymbolAddress(scratch) on device "
                         "%d failed: %s", dev, hipGetErrorString(e));
                return JINF_HIP_ERR_DEVICE;
            }
            g_scratch_base[dev].store(p, std::memory_order_release);
        }
    }
    *base = p;
    return JINF_HIP_OK;
}

}  // namespace jinf

extern "C" int jinf_attention_decode_noalloc(float* out, int ld_out, const float* q, int ld_q,
                                             const void* k_cache, const void* v_cache,
                                             int kv_type, int64_t ld_pos, int64_t ld_seq,
                                             const int32_t* lens, int n_seq, int max_ctx,
                                             int head_dim, int n_heads, int n_heads_kv,
                                             float scale, hipStream_t stream) {
    if ((!lens && n_seq > 0) || max_ctx < 0) return JINF_HIP_ERR_INVALID;
    if (n_seq > 1 && ld_seq != 0 && ld_seq < (int64_t)max_ctx * ld_pos) return JINF_HIP_ERR_INVALID;
    if (scale == 0.0f && head_dim > 0) scale = jinf::inv_sqrt_hd(head_dim);
    void* base = nullptr;
    const int st = jinf::scratch_base(&base);
    if (st != JINF_HIP_OK) return st;
    return jinf::attention_decode(out, ld_out, q, ld_q, k_cache, v_cache, kv_type, ld_pos, ld_seq,
                                  lens, max_ctx, n_seq, head_dim, n_heads, n_heads_kv, scale,
                                  jinf::AmScratch{base, 0, true}, stream);
}

// Drop-in for cuda/attention_kernel.cu:100-115: one sequence, fp32 cache
// [max_ctx][n_heads_kv][head_dim], n_past positions (n_past <= 0: nothing).
extern "C" void jinf_cuda_attention(float* output, const float* q, const float* k_cache,
                                    const float* v_cache, int head_dim, int n_heads,
                                    int n_heads_kv, int n_past, int max_ctx, hipStream_t stream) {
    if (n_past <= 0) return;
    if (head_dim <= 0 || n_heads <= 0 || n_heads_kv <= 0 || (max_ctx > 0 && n_past > max_ctx)) {
        JINF_LOG("jinf_cuda_attention: invalid argument (head_dim=%d n_heads=%d n_heads_kv=%d "
                 "n_past=%d max_ctx=%d)", head_dim, n_heads, n_heads_kv, n_past, max_ctx);
        return;
    }
    const int64_t kvw = (int64_t)n_heads_kv * head_dim;
    const int st = jinf::attention_decode(output, (int64_t)n_heads * head_dim, q,
                                          (int64_t)n_heads * head_dim, k_cache, v_cache,
                                          JINF_HIP_F32, kvw, kvw * (max_ctx > 0 ? max_ctx : n_past),
                                          nullptr, n_past, 1, head_dim, n_heads, n_heads_kv,
                                          jinf::inv_sqrt_hd(head_dim),
                                          jinf::AmScratch{nullptr, 0, false}, stream);
    if (st == JINF_HIP_ERR_INVALID)
        JINF_LOG("jinf_cuda_attention: invalid argument (head_dim=%d n_heads=%d n_heads_kv=%d)",
                 head_dim, n_heads, n_heads_kv);
}
