// Q/K/V rows of two weight formats in one launch (jinf_rmsnorm_qkv_rope's
// work for the Q4_K_M layout: q and k in Q4_K, v in Q6_K), for the decode
// engine.  Workgroups [0, nb1) run the first format's one-tile RMSNorm + RoPE
// body and the rest the second's, each exactly as its own launch would
// (matvec_body.inc), so every row's arithmetic is that of
// jinf_rmsnorm_qkv_rope.
//
// Built as a translation unit of its own, and so a code object of its own:
// compiled into matvec.hip's code object, the extra kernels slowed the
// engine's single-format Q4_0 decode step by 0.5% (1.335 -> 1.342 ms, with
// every matvec_kernel's machine code unchanged); here that object is
// byte-for-byte the one without them.
#define JINF_MATVEC_KERNELS_ONLY
#include "matvec.hip"
#include "engine_internal.h"

namespace jinf {

// The same body in a launch that serves two jobs: this job's workgroups are
// numbered bid of nblk.
template <int QT, bool ONE_TILE, int PRO, int EPI, int WV1, bool TALL = false, int XW = 28>
__device__ __forceinline__ void mv_body_shared(MvJob job, MvTheta<EPI> th, int bid, int nblk) {
#define MV_BID bid
#define MV_NBLK nblk
#include "matvec_body.inc"
#undef MV_BID
#undef MV_NBLK
}

// Q/K/V rows of two weight formats in one launch (the Q4_K_M layout: Q4_K q
// and k, Q6_K v): workgroups [0, nb1) run the first job's one-tile body and
// the rest the second's, each as its own launch would.
template <int QT1, int QT2>
__global__ __launch_bounds__(256) void matvec_qkv2_kernel(MvJob j1, MvJob j2,
                                                          MvTheta<kEpiQKV> th, int nb1) {
    if ((int)blockIdx.x < nb1)
        mv_body_shared<QT1, true, kProNorm, kEpiQKV, 4>(j1, th, blockIdx.x, nb1);
    else
        mv_body_shared<QT2, true, kProNorm, kEpiQKV, 4>(j2, th, blockIdx.x - nb1,
                                                        gridDim.x - nb1);
}

// The one-tile Q/K/V launch mv_run makes for a job with an RMSNorm
// prologue (4-wave workgroups, at most 512): fills the job's geometry and
// returns the workgroups and LDS bytes, or false where mv_run would pick
// another kernel.
template <int QT>
static bool mv_qkv_plan(MvJob& job, int cols, int* grid, size_t* shmem) {
    using F = MvFmt<QT>;
    using G = MvGroup<QT, kEpiQKV>;
    job.nb = cols / F::kElems;
    job.row_bytes = (int64_t)job.nb * F::kBytes;
    job.nt = (cols + kMvTileElems - 1) / kMvTileElems;
    if (job.nt != 1 || cols % F::kColGranule != 0 || !aligned(job.x, 16) ||
        !aligned(job.norm_w, job.norm_f16 ? 8 : 16))
        return false;
    for (int s = 0; s < 3; ++s)
        if (!aligned(job.W[s], 16)) return false;
    constexpr int xt16 = F::kPlanes ? kMvRecTile16 : 1024;
    constexpr int waves = 4;
    const int g = (G::groups(job) + waves - 1) / waves;
    *grid = g > 512 ? 512 : g;
    *shmem = ((size_t)xt16 + (size_t)waves * MvTile<QT, G::R>::kStageChunks) * 16;
    return true;
}

static bool mv_qkv_plan_any(int qtype, MvJob& job, int cols, int* grid, size_t* shmem) {
    switch (qtype) {
        case kQ4_0: return mv_qkv_plan<kQ4_0>(job, cols, grid, shmem);
        case kQ8_0: return mv_qkv_plan<kQ8_0>(job, cols, grid, shmem);
        case kQ4_K: return mv_qkv_plan<kQ4_K>(job, cols, grid, shmem);
        case kQ6_K: return mv_qkv_plan<kQ6_K>(job, cols, grid, shmem);
        default: return false;
    }
}

template <int QT1, int QT2>
static int qkv2_launch(const MvJob& j1, const MvJob& j2, const RopeTheta& th, int g1, int g2,
                       size_t shmem, hipStream_t stream) {
    return launch(matvec_qkv2_kernel<QT1, QT2>, dim3((unsigned)(g1 + g2)), dim3(256), shmem,
                  stream, j1, j2, th, g1);
}

int rmsnorm_qkv_rope_two(const void* wq, const void* wk, int qtype_qk, const void* wv,
                         int qtype_v, const float* h, const void* norm_w, int norm_type,
                         float eps, int cols, float* q_out, void* k_cache, void* v_cache,
                         int kv_type, const int32_t* pos, int max_ctx, int head_dim,
                         int n_heads, int n_heads_kv, float freq_base, hipStream_t stream,
                         bool* launched) {
    *launched = false;
    if (!norm_w || !wq || !wk || !wv || qtype_qk == qtype_v) return JINF_HIP_OK;
    MvJob j1, j2;
    bool none1 = true, none2 = true;
    int rc = qkv_job(j1, &none1, wq, wk, nullptr, qtype_qk, h, norm_w, norm_type, eps, cols,
                     q_out, k_cache, v_cache, kv_type, pos, max_ctx, head_dim, n_heads,
                     n_heads_kv, freq_base);
    if (rc == JINF_HIP_OK)
        rc = qkv_job(j2, &none2, nullptr, nullptr, wv, qtype_v, h, norm_w, norm_type, eps, cols,
                     q_out, k_cache, v_cache, kv_type, pos, max_ctx, head_dim, n_heads,
                     n_heads_kv, freq_base);
    if (rc != JINF_HIP_OK || none1 || none2) return rc;
    int g1, g2;
    size_t s1, s2;
    if (!mv_qkv_plan_any(qtype_qk, j1, cols, &g1, &s1) ||
        !mv_qkv_plan_any(qtype_v, j2, cols, &g2, &s2))
        return JINF_HIP_OK;
    RopeTheta th;
    theta_table(th, head_dim, freq_base);
    const size_t shmem = s1 > s2 ? s1 : s2;
    // the pairs of the layouts in use (a 4-bit q/k format beside a one-row v
    // format); any other pair takes one launch per format
    if (qtype_qk == kQ4_K && qtype_v == kQ6_K)
        rc = qkv2_launch<kQ4_K, kQ6_K>(j1, j2, th, g1, g2, shmem, stream);
    else if (qtype_qk == kQ4_0 && qtype_v == kQ6_K)
        rc = qkv2_launch<kQ4_0, kQ6_K>(j1, j2, th, g1, g2, shmem, stream);
    else if (qtype_qk == kQ4_0 && qtype_v == kQ8_0)
        rc = qkv2_launch<kQ4_0, kQ8_0>(j1, j2, th, g1, g2, shmem, stream);
    else if (qtype_qk == kQ4_K && qtype_v == kQ8_0)
        rc = qkv2_launch<kQ4_K, kQ8_0>(j1, j2, th, g1, g2, shmem, stream);
    else
        return JINF_HIP_OK;
    *launched = rc == JINF_HIP_OK;
    return rc;
}

}  // namespace jinf
