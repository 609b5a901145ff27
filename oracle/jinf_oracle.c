/*
 * CPU oracle for the jinf per-layer elementwise / reduction kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU kernels are
 * compared against (tests/, __graft_entry__.smoke(), and the cpu_baseline leg
 * of bench.py); the product path never calls it.
 *
 * It restates the reference's arithmetic for each kernel in plain C, with the
 * rounding points of the reference source and transcendentals evaluated in
 * fp64 (glibc) and rounded once to fp32 where the reference rounds:
 *   fp16 <-> fp32          cuda/cuda_utils.cuh:10-14, src/quant.cpp:7-45
 *   Q4_0 dequant / gather  src/quant.cpp:49-60, cuda/dequant_kernels.cu:6-21,
 *                          src/engine.cpp:170-178, 311-317
 *   RMSNorm                cuda/rmsnorm_kernel.cu:9-61
 *   residual add           cuda/matmul_kernels.cu:189-194
 *   residual -> RMSNorm    src/engine.cpp:466->487, 508->429
 *   RoPE                   cuda/rope_kernel.cu:8-50
 *   SiLU * up              cuda/silu_kernel.cu:6-18
 *   softmax                cuda/softmax_kernel.cu:8-42, cuda/attention_kernel.cu:59-87
 *   Q4_0 dequant-GEMV      cuda/matmul_kernels.cu:8-43, 198-225
 *   Q4_K / Q8_0 / Q6_K     src/quant.cpp:64-105, cuda/dequant_kernels.cu:25-110,
 *   dequant and GEMV       cuda/matmul_kernels.cu:47-185
 *   GQA decode attention   cuda/attention_kernel.cu:25-96, src/engine.cpp:446-459
 * Build with -ffp-contract=off (no FMA contraction) and without fast-math.
 *
 * fp16 storage: every stored value is fl16(fl32(expression)) with
 * round-to-nearest-even and subnormals kept.
 *
 * Rows are split over OpenMP threads only for the CPU baseline timing; each
 * row's arithmetic is sequential and identical for any thread count.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define JO_F32 0
#define JO_F16 1

static int jo_threads = 1;

void jo_set_threads(int n) { jo_threads = n < 1 ? 1 : n; }
int jo_get_threads(void) { return jo_threads; }

/* ---- binary16 <-> binary32 (IEEE 754 definitions) ---- */

/* Exact widening; same results as src/quant.cpp:7-45. */
float jo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        const float v = ldexpf((float)m, -24); /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31)
        bits = sign | 0x7F800000u | (m << 13);
    else
        bits = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even narrowing, subnormals kept, overflow to Inf,
 * NaN stays NaN (quiet, top payload bits kept). */
uint16_t jo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 */
    if (ax >= 0x38800000u) {                                 /* >= 2^-14: normal */
        const uint32_t m = ax - 0x38000000u;                 /* rebias 127 -> 15 */
        return (uint16_t)(sign | ((m + 0x0FFFu + ((m >> 13) & 1u)) >> 13));
    }
    const uint32_t e = ax >> 23;
    if (e < 102) return sign; /* below 2^-25: rounds to zero */
    const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e; /* units of 2^-24 */
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

void jo_f16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = jo_f16_to_f32(in[i]);
}

void jo_f32_to_f16_n(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = jo_f32_to_f16(in[i]);
}

static inline float ld_act(const void* p, int type, int64_t i) {
    return type == JO_F16 ? jo_f16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

static inline void st_act(void* p, int type, int64_t i, float v) {
    if (type == JO_F16)
        ((uint16_t*)p)[i] = jo_f32_to_f16(v);
    else
        ((float*)p)[i] = v;
}

static inline float round_act(int type, float v) {
    return type == JO_F16 ? jo_f16_to_f32(jo_f32_to_f16(v)) : v;
}

/* ---- Q4_0 (src/quant.cpp:49-60; block layout include/jinf/quant.h:30-36) ---- */

static void q4_0_block(const uint8_t* blk, int type, void* out, int64_t o) {
    const uint16_t dbits = (uint16_t)(blk[0] | (blk[1] << 8)); /* little-endian */
    const float d = jo_f16_to_f32(dbits);
    for (int j = 0; j < 16; ++j) {
        const uint8_t b = blk[2 + j];
        const int v0 = (int)(b & 0x0F) - 8;
        const int v1 = (int)(b >> 4) - 8;
        st_act(out, type, o + 2 * j, (float)v0 * d);
        st_act(out, type, o + 2 * j + 1, (float)v1 * d);
    }
}

/* Contiguous blocks to fp32: the reference CPU path jinf_dequantize_q4_0. */
void jo_dequant_q4_0(const uint8_t* blocks, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; ++b) q4_0_block(blocks + 18 * (int64_t)b, JO_F32, out, 32 * (int64_t)b);
}

/* Token-embedding gather (src/engine.cpp:311-317): row ids[i] of a table of
 * n_vocab rows of n_embd/32 blocks.  ids == NULL means row i.  Out-of-range ids
 * give a +0.0 row (the GPU contract; the reference does not check). */
void jo_embed_q4_0(void* out, int out_type, int64_t ld_out, const uint8_t* table, int n_vocab,
                   int n_embd, const int32_t* ids, int n_ids) {
    const int nb = n_embd / 32;
    const int64_t row_bytes = (int64_t)nb * 18;
#pragma omp parallel for num_threads(jo_threads) schedule(static)
    for (int i = 0; i < n_ids; ++i) {
        const int id = ids ? ids[i] : i;
        const int64_t o = (int64_t)i * ld_out;
        if (id < 0 || id >= n_vocab) {
            for (int e = 0; e < n_embd; ++e) st_act(out, out_type, o + e, 0.0f);
            continue;
        }
        const uint8_t* row = table + (int64_t)id * row_bytes;
        for (int b = 0; b < nb; ++b) q4_0_block(row + 18 * (int64_t)b, out_type, out, o + 32 * (int64_t)b);
    }
}

/* ---- RMSNorm (cuda/rmsnorm_kernel.cu:9-61) ---- */

/* rs = 1/sqrt(fl32(fl32(ss)/n) + eps), sqrt and divide in fp64, rounded once. */
static float rms_scale(double ss, int n, float eps) {
    const float m = (float)ss / (float)n;
    const float t = m + eps;
    return (float)(1.0 / sqrt((double)t));
}

static void norm_row(void* out, int64_t oo, const float* h, const void* w, int wt, int n,
                     float eps, int act) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)h[i] * (double)h[i];
    const float rs = rms_scale(ss, n, eps);
    for (int i = 0; i < n; ++i) st_act(out, act, oo + i, (h[i] * rs) * ld_act(w, wt, i));
}

/* out[r] = rmsnorm(in[r]) * w.  Sum of squares sequential in fp64. */
void jo_rmsnorm_rows(void* out, int64_t ld_out, const void* in, int64_t ld_in, const void* w,
                     int n_rows, int n, float eps, int act, int wt) {
#pragma omp parallel num_threads(jo_threads)
    {
        float hbuf[65536];
#pragma omp for schedule(static)
        for (int r = 0; r < n_rows; ++r) {
            for (int i = 0; i < n; ++i) hbuf[i] = ld_act(in, act, (int64_t)r * ld_in + i);
            norm_row(out, (int64_t)r * ld_out, hbuf, w, wt, n, eps, act);
        }
    }
}

/* residual[r] = round(residual[r] + delta[r]) (stored); out[r] = rmsnorm(residual[r]) * w. */
void jo_residual_rmsnorm_rows(void* out, int64_t ld_out, void* res, int64_t ld_res,
                              const void* delta, int64_t ld_delta, const void* w, int n_rows,
                              int n, float eps, int act, int wt) {
#pragma omp parallel num_threads(jo_threads)
    {
        float hbuf[65536];
#pragma omp for schedule(static)
        for (int r = 0; r < n_rows; ++r) {
            for (int i = 0; i < n; ++i) {
                const float v = ld_act(res, act, (int64_t)r * ld_res + i) +
                                ld_act(delta, act, (int64_t)r * ld_delta + i);
                st_act(res, act, (int64_t)r * ld_res + i, v);
                hbuf[i] = round_act(act, v);
            }
            norm_row(out, (int64_t)r * ld_out, hbuf, w, wt, n, eps, act);
        }
    }
}

/* The reference kernel's own fp32 summation order for one row: per-thread
 * strided partials over T = min(n,1024) rounded up to 32 threads, each
 * accumulated as fma(v, v, acc) (nvcc contracts sum += v*v), then the 32-lane
 * shfl_down tree per warp and the same tree over the warp partials
 * (cuda/cuda_utils.cuh:18-49, cuda/rmsnorm_kernel.cu:16-22,67-69).
 * Returns the fp32 sum of squares; used to bound how far the reference's
 * rounding of ss can sit from the fp64 sum used above. */
float jo_ref_order_sumsq(const float* x, int n) {
    int T = n < 1024 ? n : 1024;
    T = (T + 31) / 32 * 32;
    if (T > 1024) T = 1024;
    float part[1024];
    for (int t = 0; t < T; ++t) {
        float acc = 0.0f;
        for (int i = t; i < n; i += T) acc = fmaf(x[i], x[i], acc);
        part[t] = acc;
    }
    const int nw = (T + 31) / 32;
    float warp[32];
    for (int w = 0; w < nw; ++w) {
        float v[32];
        for (int l = 0; l < 32; ++l) v[l] = part[32 * w + l];
        for (int off = 16; off > 0; off >>= 1)
            for (int l = 0; l < 32; ++l) v[l] = v[l] + (l + off < 32 ? v[l + off] : 0.0f);
        warp[w] = v[0];
    }
    float v[32];
    for (int l = 0; l < 32; ++l) v[l] = l < nw ? warp[l] : 0.0f;
    for (int off = 16; off > 0; off >>= 1)
        for (int l = 0; l < 32; ++l) v[l] = v[l] + (l + off < 32 ? v[l + off] : 0.0f);
    return v[0];
}

/* ---- residual add (cuda/matmul_kernels.cu:189-194) ---- */

void jo_residual_add(void* a, const void* b, int64_t n, int act) {
#pragma omp parallel for num_threads(jo_threads) schedule(static)
    for (int64_t i = 0; i < n; ++i) st_act(a, act, i, ld_act(a, act, i) + ld_act(b, act, i));
}

/* ---- RoPE (cuda/rope_kernel.cu:8-50) ---- */

/* theta_i = fl32(base^e), e = fl32(fl32(-2*i)/hd) as the reference forms it. */
float jo_rope_theta(float base, int i, int head_dim) {
    volatile float e = -2.0f * (float)i;
    e = e / (float)head_dim;
    return (float)pow((double)base, (double)e);
}

static void rope_head(void* p, int act, int64_t o, int head_dim, const float* c, const float* s) {
    for (int i = 0; i < head_dim / 2; ++i) {
        const float x0 = ld_act(p, act, o + 2 * i);
        const float x1 = ld_act(p, act, o + 2 * i + 1);
        st_act(p, act, o + 2 * i, x0 * c[i] - x1 * s[i]);
        st_act(p, act, o + 2 * i + 1, x0 * s[i] + x1 * c[i]);
    }
}

/* In place over n_tokens tokens; token t uses positions[t] (or pos0 + t). */
void jo_rope_rows(void* q, int64_t ld_q, void* k, int64_t ld_k, const int32_t* positions,
                  int pos0, int n_tokens, int head_dim, int n_heads, int n_heads_kv, float base,
                  int act) {
    float theta[4096];
    for (int i = 0; i < head_dim / 2; ++i) theta[i] = jo_rope_theta(base, i, head_dim);
#pragma omp parallel num_threads(jo_threads)
    {
        float c[4096], s[4096];
#pragma omp for schedule(static)
        for (int t = 0; t < n_tokens; ++t) {
            const int pos = positions ? positions[t] : pos0 + t;
            for (int i = 0; i < head_dim / 2; ++i) {
                const float a = (float)pos * theta[i];
                c[i] = (float)cos((double)a);
                s[i] = (float)sin((double)a);
            }
            for (int h = 0; h < n_heads; ++h)
                rope_head(q, act, (int64_t)t * ld_q + (int64_t)h * head_dim, head_dim, c, s);
            for (int h = 0; h < n_heads_kv; ++h)
                rope_head(k, act, (int64_t)t * ld_k + (int64_t)h * head_dim, head_dim, c, s);
        }
    }
}

/* ---- SiLU(gate) * up (cuda/silu_kernel.cu:6-18) ---- */

void jo_swiglu(void* out, const void* gate, const void* up, int64_t n, int act) {
#pragma omp parallel for num_threads(jo_threads) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float g = ld_act(gate, act, i);
        const float e = (float)exp(-(double)g);
        const float silu = g / (1.0f + e);
        st_act(out, act, i, silu * ld_act(up, act, i));
    }
}

/* ---- softmax (cuda/softmax_kernel.cu:8-42, cuda/attention_kernel.cu:59-87) ---- */

/* Row r has live length L = lens ? clamp(lens[r / rows_per_len], 0, n_cols)
 * : n_cols.  s = scale * x; y_j = fl32(exp(s_j - m)) * fl32(1 / sum), with the
 * sum of the rounded exponentials accumulated in fp64.  j >= L untouched. */
void jo_softmax_rows(float* out, int64_t ld_out, const float* in, int64_t ld_in, int n_rows,
                     int n_cols, const int32_t* lens, int rows_per_len, float scale) {
#pragma omp parallel for num_threads(jo_threads) schedule(dynamic, 16)
    for (int r = 0; r < n_rows; ++r) {
        int L = n_cols;
        if (lens) {
            L = lens[r / rows_per_len];
            L = L < 0 ? 0 : (L > n_cols ? n_cols : L);
        }
        if (L == 0) continue;
        const float* x = in + (int64_t)r * ld_in;
        float* y = out + (int64_t)r * ld_out;
        float m = -INFINITY;
        for (int j = 0; j < L; ++j) m = fmaxf(m, x[j] * scale);
        double sum = 0.0;
        for (int j = 0; j < L; ++j) sum += (double)(float)exp((double)(x[j] * scale - m));
        const float inv = 1.0f / (float)sum;
        for (int j = 0; j < L; ++j) y[j] = (float)exp((double)(x[j] * scale - m)) * inv;
    }
}

/* ---- Q4_0 dequant-GEMV (cuda/matmul_kernels.cu:8-43, :198-225) ---- */

/* y[r] = sum_j ((q_j - 8) * d) * x[j]; every product is exact in fp64 (a
 * 15-bit weight times a 24-bit x) and the sum is accumulated in fp64 in
 * column order, then rounded once.  abs_y (optional) receives
 * sum_j |w_j * x_j|, the scale of the dot product's rounding error. */
void jo_matvec_q4_0(const uint8_t* W, const float* x, float* y, double* abs_y, int rows,
                    int cols) {
    const int nb = cols / 32;
    const int64_t row_bytes = (int64_t)nb * 18;
#pragma omp parallel for num_threads(jo_threads) schedule(static)
    for (int r = 0; r < rows; ++r) {
        double acc = 0.0, aabs = 0.0;
        const uint8_t* row = W + (int64_t)r * row_bytes;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = row + 18 * (int64_t)b;
            const double d = (double)jo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int j = 0; j < 16; ++j) {
                const uint8_t byte = blk[2 + j];
                const double t0 = (double)((int)(byte & 0x0F) - 8) * d * (double)x[32 * b + 2 * j];
                const double t1 = (double)((int)(byte >> 4) - 8) * d * (double)x[32 * b + 2 * j + 1];
                acc += t0 + t1;
                aabs += fabs(t0) + fabs(t1);
            }
        }
        y[r] = (float)acc;
        if (abs_y) abs_y[r] = aabs;
    }
}

/* ---- Q4_K, Q8_0, Q6_K (block layouts include/jinf/quant.h:38-68) ---- */

/* The reference's own 6-bit unpacking of the 12 scale bytes into 8 scales and
 * 8 mins (src/quant.cpp:70-75, cuda/matmul_kernels.cu:65-70): sub-blocks 0-3
 * take the low 6 bits of bytes 0-3 (scales) and 4-7 (mins); sub-blocks 4-7
 * take a nibble of bytes 8-11 as their HIGH four bits and the top two bits of
 * bytes 0-3 / 4-7 as their low two. */
static void q4_K_scales(const uint8_t* s, int sc[8], int mn[8]) {
    for (int i = 0; i < 4; ++i) {
        sc[i] = s[i] & 0x3F;
        mn[i] = s[i + 4] & 0x3F;
        sc[i + 4] = ((s[i + 8] & 0x0F) << 2) | (s[i] >> 6);
        mn[i + 4] = ((s[i + 8] >> 4) << 2) | (s[i + 4] >> 6);
    }
}

/* One 144-byte Q4_K super-block (256 values): d, dmin (binary16), scales[12],
 * qs[128]; element 2i of sub-block sb is the low nibble of qs[16 sb + i], 2i+1
 * the high nibble.  w = sub_d * q - sub_min with sub_d = d * sc and
 * sub_min = dmin * mn; both products and sub_d * q are exact in fp32, so the
 * subtraction is the only rounding (with or without FMA contraction). */
static void q4_K_block(const uint8_t* blk, float* out) {
    const float d = jo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const float dmin = jo_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    int sc[8], mn[8];
    q4_K_scales(blk + 4, sc, mn);
    for (int sb = 0; sb < 8; ++sb) {
        const float sub_d = d * (float)sc[sb];
        const float sub_min = dmin * (float)mn[sb];
        for (int i = 0; i < 16; ++i) {
            const uint8_t b = blk[16 + 16 * sb + i];
            out[32 * sb + 2 * i] = sub_d * (float)(b & 0x0F) - sub_min;
            out[32 * sb + 2 * i + 1] = sub_d * (float)(b >> 4) - sub_min;
        }
    }
}

/* One 34-byte Q8_0 block: d (binary16), 32 int8; w = q * d, exact. */
static void q8_0_block(const uint8_t* blk, float* out) {
    const float d = jo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)blk[2 + i] * d;
}

/* One 210-byte Q6_K super-block (cuda/dequant_kernels.cu:82-110): ql[128],
 * qh[64], int8 scales[16], then d (binary16) at byte 208.  Element e:
 * low four bits from ql[e/2] (low nibble for even e), high two bits from
 * qh[e/4] at bit 2*(e%4); w = (d * scales[e/16]) * (q6 - 32).  d * scale has
 * at most 18 significant bits and |q6 - 32| <= 32, so both products are exact. */
static void q6_K_block(const uint8_t* blk, float* out) {
    const float d = jo_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
    for (int e = 0; e < 256; ++e) {
        const uint8_t l = blk[e / 2];
        const int lo = (e & 1) ? (l >> 4) : (l & 0x0F);
        const int hi = (blk[128 + e / 4] >> (2 * (e % 4))) & 0x03;
        const int q6 = lo | (hi << 4);
        out[e] = d * (float)(int8_t)blk[192 + e / 16] * (float)(q6 - 32);
    }
}

/* Block geometry of a supported qtype (include/jinf/quant.h:8-24 codes):
 * returns values per block and sets *bytes, or 0 for an unsupported type. */
int jo_qtype_geometry(int qtype, int* bytes) {
    switch (qtype) {
        case 2: *bytes = 18; return 32;    /* Q4_0 */
        case 8: *bytes = 34; return 32;    /* Q8_0 */
        case 12: *bytes = 144; return 256; /* Q4_K */
        case 14: *bytes = 210; return 256; /* Q6_K */
        default: *bytes = 0; return 0;
    }
}

static void dequant_block(int qtype, const uint8_t* blk, float* out) {
    switch (qtype) {
        case 2: q4_0_block(blk, JO_F32, out, 0); break;
        case 8: q8_0_block(blk, out); break;
        case 12: q4_K_block(blk, out); break;
        case 14: q6_K_block(blk, out); break;
        default: break;
    }
}

/* n_blocks contiguous blocks of qtype to fp32 (the reference's
 * jinf_dequantize_q4_K / _q8_0 and the GPU launchers
 * jinf_cuda_dequantize_q4_K / _q8_0 / _q6_K). */
void jo_dequant(int qtype, const uint8_t* blocks, float* out, int n_blocks) {
    int bytes;
    const int elems = jo_qtype_geometry(qtype, &bytes);
    if (!elems) return;
    for (int b = 0; b < n_blocks; ++b)
        dequant_block(qtype, blocks + (int64_t)bytes * b, out + (int64_t)elems * b);
}

/* y[r] = sum_j w[r, j] * x[j] for any supported qtype (cuda/matmul_kernels.cu
 * :8-185): each row is dequantized exactly as above, the products are formed
 * and summed in fp64 in column order and rounded once; abs_y (optional)
 * receives sum_j |w_j x_j|. */
void jo_matvec(int qtype, const uint8_t* W, const float* x, float* y, double* abs_y, int rows,
               int cols) {
    int bytes;
    const int elems = jo_qtype_geometry(qtype, &bytes);
    if (!elems || cols % elems) return;
    const int nb = cols / elems;
    const int64_t row_bytes = (int64_t)nb * bytes;
#pragma omp parallel num_threads(jo_threads)
    {
        float wblk[256];
#pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            double acc = 0.0, aabs = 0.0;
            const uint8_t* row = W + (int64_t)r * row_bytes;
            for (int b = 0; b < nb; ++b) {
                dequant_block(qtype, row + (int64_t)bytes * b, wblk);
                for (int j = 0; j < elems; ++j) {
                    const double t = (double)wblk[j] * (double)x[(int64_t)elems * b + j];
                    acc += t;
                    aabs += fabs(t);
                }
            }
            y[r] = (float)acc;
            if (abs_y) abs_y[r] = aabs;
        }
    }
}

/* ---- GQA decode attention (cuda/attention_kernel.cu:25-96) ---- */

/* For every sequence s and query head h (kv head h / (n_heads / n_heads_kv)):
 *   score_t = (q_h . k_t) * scale             t = 0 .. lens[s] - 1
 *   p_t     = exp(score_t - max) / sum_u exp(score_u - max)
 *   out_h   = sum_t p_t * v_t
 * evaluated entirely in fp64 from the stored fp32/fp16 values and rounded to
 * fp32 once (the reference rounds the dot, the exp, the sum and every
 * accumulation to fp32; the GPU tolerance covers that).  The cache of sequence
 * s, position t, kv head j starts at element s * ld_seq + t * ld_pos +
 * j * head_dim.  abs_out (optional) receives sum_t p_t |v_t[d]|, the scale of
 * the output's rounding error.  Positions at or past lens[s] are never read. */
void jo_attention(float* out, int64_t ld_out, const float* q, int64_t ld_q, const void* k,
                  const void* v, int kv_type, int64_t ld_pos, int64_t ld_seq,
                  const int32_t* lens, int n_seq, int head_dim, int n_heads, int n_heads_kv,
                  double scale, double* abs_out) {
    const int group = n_heads / n_heads_kv;
#pragma omp parallel num_threads(jo_threads)
    {
        double acc[1024], aabs[1024];
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int s = 0; s < n_seq; ++s) {
            for (int h = 0; h < n_heads; ++h) {
                const int len = lens[s];
                const int j = h / group;
                const float* qh = q + (int64_t)s * ld_q + (int64_t)h * head_dim;
                double m = -INFINITY;
                for (int t = 0; t < len; ++t) {
                    const int64_t o = (int64_t)s * ld_seq + (int64_t)t * ld_pos + (int64_t)j * head_dim;
                    double dot = 0.0;
                    for (int d = 0; d < head_dim; ++d) dot += (double)qh[d] * (double)ld_act(k, kv_type, o + d);
                    const double sc = dot * scale;
                    if (sc > m) m = sc;
                }
                for (int d = 0; d < head_dim; ++d) acc[d] = aabs[d] = 0.0;
                double l = 0.0;
                for (int t = 0; t < len; ++t) {
                    const int64_t o = (int64_t)s * ld_seq + (int64_t)t * ld_pos + (int64_t)j * head_dim;
                    double dot = 0.0;
                    for (int d = 0; d < head_dim; ++d) dot += (double)qh[d] * (double)ld_act(k, kv_type, o + d);
                    const double e = exp(dot * scale - m);
                    l += e;
                    for (int d = 0; d < head_dim; ++d) {
                        const double vv = (double)ld_act(v, kv_type, o + d);
                        acc[d] += e * vv;
                        aabs[d] += e * fabs(vv);
                    }
                }
                float* oh = out + (int64_t)s * ld_out + (int64_t)h * head_dim;
                double* ah = abs_out ? abs_out + ((int64_t)s * n_heads + h) * head_dim : 0;
                for (int d = 0; d < head_dim; ++d) {
                    oh[d] = len > 0 ? (float)(acc[d] / l) : 0.0f;
                    if (ah) ah[d] = len > 0 ? aabs[d] / l : 0.0;
                }
            }
        }
    }
}
