// Q4_0 dequant + matrix-vector product for gfx950.
//
// Semantics (reference cuda/matmul_kernels.cu:8-43 and the launcher
// :198-225): W is [rows, cols] in GGUF Q4_0 blocks along the columns
// (include/jinf/quant.h:30-36, jinf's interleaved element order: element 2j
// of a block is the low nibble of qs[j], element 2j+1 the high nibble);
//   y[row] = sum_j ((q_j - 8) * d_block(j)) * x[j]
// in fp32.  The summation order is not the reference's (its per-thread
// strided loop and warp tree); results agree to fp32 rounding of the dot
// product.
//
// Design: batch-1 decode is HBM-bound on the 18-byte blocks (0.5625 B per
// weight), so every weight byte is read once, with nontemporal coalesced
// 16-byte loads, and x is kept out of the per-row traffic:
//   - work items are R rows x one column tile of 128 blocks (4096 columns,
//     2304 bytes of a row); a wave owns whole groups of R rows and walks their
//     tiles, prefetching the next item's bytes into registers while it
//     computes the current one;
//   - the tile bytes go through the wave's own LDS region, so each lane reads
//     back two whole consecutive blocks (36 bytes: bank-conflict free);
//   - x is staged once per workgroup in LDS; a lane keeps the 64 x values of
//     its two blocks in registers (for the whole kernel when the matrix is
//     one tile wide) and reuses them for all R rows;
//   - dequantisation is folded into the dot product (fp16-denormal nibbles and
//     v_fma_mix_f32, see q4_dot32_mix); the block's -8 offset and scale d are
//     applied once per block;
//   - each row's lane partials meet in a DPP wave reduction.
#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/kernels.h"

namespace jinf {

constexpr int kMvBPL = 2;                 // consecutive blocks per lane per tile
constexpr int kMvTile = kWave * kMvBPL;   // blocks per column tile
constexpr int kMvWaves = 4;               // waves per workgroup

// Dot of one block's 32 nibbles (4 words, jinf order) with x[0..31]: returns
// sum_j (q_j - 8) * x_j, accumulated with fma in element order.
__device__ __forceinline__ float q4_dot32(const uint32_t (&qw)[4], const float* x) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int w = (int)(qw[i] ^ 0x88888888u);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int lo = __builtin_amdgcn_sbfe(w, 8 * m, 4);      // q - 8, element 8i+2m
            const int hi = __builtin_amdgcn_sbfe(w, 8 * m + 4, 4);  // element 8i+2m+1
            s = fmaf((float)lo, x[8 * i + 2 * m], s);
            s = fmaf((float)hi, x[8 * i + 2 * m + 1], s);
        }
    }
    return s;
}

// Bytes of one row's column tile (128 blocks), and its 16-byte chunks.
constexpr int kMvTileBytes = kMvTile * 18;       // 2304
constexpr int kMvChunks = kMvTileBytes / 16;     // 144
constexpr int kMvChunksPerLane = 3;              // ceil(144 / 64)
// Chunk slots past a row's 144 that lanes 16..63 write in the third pass.
constexpr int kMvPad = kWave * kMvChunksPerLane - kMvChunks;  // 48
// LDS staging per wave: R rows of 144 chunks, then the pad.
__host__ __device__ constexpr int mv_stage_chunks(int R) { return R * kMvChunks + kMvPad; }

// The nibbles are multiplied as fp16 denormals: masking a word with
// 0x000F000F leaves two halves whose bits are nibbles, i.e. the fp16 values
// q * 2^-24 exactly; masking with 0x00F000F0 gives (16 q) * 2^-24.  One
// v_fma_mix_f32 per weight then accumulates (q * 2^-24 * scale) * x' in fp32
// with a single rounding, where x' = x / scale holds the position's power of
// two (exact).  Word i of a block holds elements 8i..8i+7, element 8i+n in
// bits 4n..4n+3 (jinf order), so
//   w & 0x000F000F        -> elements 8i+0 (lo half), 8i+4 (hi half), scale 1
//   w & 0x00F000F0        -> 8i+1, 8i+5, scale 16
//   (w >> 8) & 0x000F000F -> 8i+2, 8i+6, scale 1
//   (w >> 8) & 0x00F000F0 -> 8i+3, 8i+7, scale 16
// (5 bit operations per 8 weights).  The lane's x registers are stored
// pre-divided by 16 at odd element positions.
typedef _Float16 mv_half2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float mix2(uint32_t h, float xlo, float xhi, float acc) {
    const mv_half2 v = __builtin_bit_cast(mv_half2, h);
    acc = fmaf((float)v.x, xlo, acc);
    return fmaf((float)v.y, xhi, acc);
}

// 2^-24 * sum_j q_j * x_j over one block (q unsigned 0..15) from its 4 words
// and the block's 32 pre-scaled x values.
__device__ __forceinline__ float q4_dot32_mix(const uint32_t (&qw)[4], const float* xp) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = qw[i];
        const uint32_t v = w >> 8;
        const float* xi = xp + 8 * i;
        s = mix2(w & 0x000F000Fu, xi[0], xi[4], s);
        s = mix2(w & 0x00F000F0u, xi[1], xi[5], s);
        s = mix2(v & 0x000F000Fu, xi[2], xi[6], s);
        s = mix2(v & 0x00F000F0u, xi[3], xi[7], s);
    }
    return s;
}

// Two blocks per lane from the wave's staged tile bytes:
// d0 * (sum q x - 8 sum x) + d1 * (...) for blocks b0, b0+1, given the
// pre-scaled x (xp) and the plain x sums xs0, xs1 of the two blocks.  The
// 2^-24 of the denormal products is returned to d (d * 2^24, exact); the -8
// offset is one fma per block, whose rounding stays at the scale of
// sum |q x|, far inside the dot product's tolerance.
__device__ __forceinline__ float q4_pair(const uint32_t* l, const float* xp, float xs0,
                                         float xs1) {
    uint32_t D[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) D[i] = l[i];
    const float d0 = h2f((uint16_t)(D[0] & 0xFFFFu)) * 16777216.0f;
    const float d1 = h2f((uint16_t)(D[4] >> 16)) * 16777216.0f;
    const uint32_t q0[4] = {__builtin_amdgcn_alignbit(D[1], D[0], 16),
                            __builtin_amdgcn_alignbit(D[2], D[1], 16),
                            __builtin_amdgcn_alignbit(D[3], D[2], 16),
                            __builtin_amdgcn_alignbit(D[4], D[3], 16)};
    const uint32_t q1[4] = {D[5], D[6], D[7], D[8]};
    constexpr float kOff = -8.0f / 16777216.0f;  // -8 * 2^-24
    const float s0 = fmaf(kOff, xs0, q4_dot32_mix(q0, xp));
    const float s1 = fmaf(kOff, xs1, q4_dot32_mix(q1, xp + 32));
    return fmaf(d1, s1, d0 * s0);
}

// x tile layout in LDS: tile t holds 1024 float4 (4096 floats); lane l's 16
// float4 (its two blocks) sit in row l with the column XOR-swizzled by l & 15,
// so the 16 lanes of one LDS pass read 16 distinct bank groups.
__device__ __forceinline__ int mv_xslot(int tile, int l, int j) {
    return (tile << 10) + (l << 4) + (j ^ (l & 15));
}

// Work is split into items (R rows, one 128-block column tile).  Each wave
// takes whole groups of R rows (groups g, g + stride, ...) and walks their
// tiles in order, so a row's partial sums stay in the wave's registers until
// its last tile.  The next item's weights are loaded one item ahead with
// coalesced 16-byte loads (ping-pong registers), staged in the wave's own LDS
// region and read back as two whole blocks per lane.  x is staged once per
// workgroup in LDS (swizzled) and copied to registers per tile (once per
// kernel when the matrix is a single tile wide).  The wave's LDS accesses
// execute in order; the fences keep the compiler from moving the read-back
// above the stores.  The only workgroup barrier follows the x staging.
template <int R, bool ONE_TILE>
__global__ __launch_bounds__(ONE_TILE ? 256 : 512) void matvec_q4_0_kernel(
    const uint8_t* __restrict__ W, int64_t row_bytes, const float* __restrict__ x,
    float* __restrict__ y, int rows, int nb, int nt) {
    extern __shared__ uint4 lds[];
    float4* xl = reinterpret_cast<float4*>(lds);
    const int waves = blockDim.x / kWave;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    uint4* stage = lds + (nt << 10) + wave * mv_stage_chunks(R);
    const int n_groups = (rows + R - 1) / R;
    const int stride = gridDim.x * waves;
    if (ONE_TILE) nt = 1;

    using Buf = uint4[R][kMvChunksPerLane];
    auto fetch = [&](int g, int t, Buf& buf) {
        const int tb = t * kMvTile;
        const int nbt = nb - tb < kMvTile ? nb - tb : kMvTile;
        const int nchunk = nbt * 18 / 16;  // nbt % 8 == 0
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = g * R + r < rows ? g * R + r : rows - 1;
            const uint8_t* src = W + (int64_t)row * row_bytes + (int64_t)tb * 18;
#pragma unroll
            for (int k = 0; k < kMvChunksPerLane; ++k) {
                // Lanes past the tile's end re-read its last chunk (never staged).
                const int c = lane + kWave * k < nchunk ? lane + kWave * k : nchunk - 1;
                buf[r][k] = ld16<true>(src + 16 * c);
            }
        }
    };
    auto advance = [&](int& g, int& t) {
        if (ONE_TILE) {
            g += stride;
        } else if (++t == nt) {
            t = 0;
            g += stride;
        }
    };

    int g0 = blockIdx.x * waves + wave, t0 = 0;
    uint4 bufA[R][kMvChunksPerLane];
    uint4 bufB[R][kMvChunksPerLane];
    if (g0 < n_groups) fetch(g0, t0, bufA);

    // Stage x (zero past the last block) while the first weights are in flight.
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (int f = threadIdx.x; f < (nt << 10); f += blockDim.x) {
        const float4 v = f < nb * 8 ? x4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
        xl[mv_xslot(f >> 10, (f >> 4) & 63, f & 15)] = v;
    }
    __syncthreads();
    if (g0 >= n_groups) return;

    float xv[kMvBPL * 32];
    float xs0 = 0.0f, xs1 = 0.0f;
    auto load_x = [&](int t) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float4 v = xl[mv_xslot(t, lane, j)];
            xv[4 * j] = v.x; xv[4 * j + 1] = v.y; xv[4 * j + 2] = v.z; xv[4 * j + 3] = v.w;
        }
        xs0 = 0.0f;
        xs1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            xs0 += xv[i];
            xs1 += xv[32 + i];
        }
#pragma unroll
        for (int i = 1; i < 64; i += 2) xv[i] *= 0.0625f;  // odd positions: x / 16
    };
    if (ONE_TILE) load_x(0);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    auto process = [&](int g, int t, const Buf& buf) {
        if (!ONE_TILE) load_x(t);
        const bool live = t * kMvTile + lane * kMvBPL < nb;
        // Every lane writes every chunk (no branch, so no load is left
        // pending on a skipped path).  The third pass goes first: its slots
        // past 144 land on the next row's first 48 chunks, which the first
        // pass then overwrites (a wave's LDS writes complete in order), and
        // the last row's on the pad.
#pragma unroll
        for (int r = 0; r < R; ++r) stage[r * kMvChunks + lane + 2 * kWave] = buf[r][2];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < 2; ++k) stage[r * kMvChunks + lane + kWave * k] = buf[r][k];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t* l = reinterpret_cast<const uint32_t*>(stage + r * kMvChunks) + 9 * lane;
            if (live) acc[r] += q4_pair(l, xv, xs0, xs1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (t == nt - 1) {  // group complete: reduce and store its rows
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v = wave_sum_f32(acc[r]);
                if (lane == 0 && g * R + r < rows) y[g * R + r] = v;
                acc[r] = 0.0f;
            }
        }
    };

    // The last item leaves through its own branch, so on the main path the
    // prefetch is unconditional and the compiler's wait counts stay exact
    // (a conditional load makes it wait for every outstanding load).
    int g1 = g0, t1 = t0;
    while (true) {
        advance(g1, t1);
        if (g1 >= n_groups) {
            process(g0, t0, bufA);
            break;
        }
        fetch(g1, t1, bufB);
        process(g0, t0, bufA);
        g0 = g1;
        t0 = t1;
        advance(g1, t1);
        if (g1 >= n_groups) {
            process(g0, t0, bufB);
            break;
        }
        fetch(g1, t1, bufA);
        process(g0, t0, bufB);
        g0 = g1;
        t0 = t1;
    }
}

// Any block count / 2-byte alignment: one wave per row, one block per lane
// step, 16-bit loads, x read per element.
__global__ __launch_bounds__(kMvWaves * kWave) void matvec_q4_0_any_kernel(
    const uint8_t* __restrict__ W, int64_t row_bytes, const float* __restrict__ x,
    float* __restrict__ y, int rows, int nb) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * kMvWaves + threadIdx.x / kWave;
    if (row >= rows) return;
    float acc = 0.0f;
    for (int b = lane; b < nb; b += kWave) {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(W + row * row_bytes + (int64_t)b * 18);
        const float d = h2f(p[0]);
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = (uint32_t)p[1 + 2 * i] | ((uint32_t)p[2 + 2 * i] << 16);
        acc = fmaf(d, q4_dot32(q, x + 32 * b), acc);
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, kWave);
    if (lane == 0) y[row] = acc;
}

// Widest matrix served by the tiled kernel: x for every tile must fit in LDS
// next to the weight staging of 8 waves (7 tiles = 28672 columns:
// 112 KiB + 8 * 5376 B).
constexpr int kMvMaxTiles = 7;

// Launch the tiled kernel with R rows per item and at most grid_cap
// workgroups.  Single-tile matrices use 4 independent waves per workgroup;
// wider ones 8 waves sharing one copy of x.
template <int R>
static int mv_launch(const void* w, const float* x, float* y, int rows, int cols, int grid_cap,
                     hipStream_t stream) {
    const int nb = cols / 32;
    const int nt = (nb + kMvTile - 1) / kMvTile;
    if (nt > kMvMaxTiles) return JINF_HIP_ERR_INVALID;
    const int waves = nt == 1 ? 4 : 8;
    const int groups = (rows + R - 1) / R;
    int grid = (groups + waves - 1) / waves;
    if (grid > grid_cap) grid = grid_cap;
    const size_t shmem = ((size_t)nt * 1024 + (size_t)waves * mv_stage_chunks(R)) * 16;
    const uint8_t* W = static_cast<const uint8_t*>(w);
    if (nt == 1)
        return launch(matvec_q4_0_kernel<R, true>, dim3(grid), dim3(waves * kWave), shmem,
                      stream, W, (int64_t)nb * 18, x, y, rows, nb, nt);
    return launch(matvec_q4_0_kernel<R, false>, dim3(grid), dim3(waves * kWave), shmem, stream,
                  W, (int64_t)nb * 18, x, y, rows, nb, nt);
}

static int matvec_q4_0(const void* w, const float* x, float* y, int rows, int cols,
                       hipStream_t stream) {
    if (rows < 0 || cols < 0) return JINF_HIP_ERR_INVALID;
    if (rows == 0 || cols == 0) return JINF_HIP_OK;
    if (!w || !x || !y || cols % 32 != 0) return JINF_HIP_ERR_INVALID;
    if (!aligned(w, 2) || !aligned(x, 4) || !aligned(y, 4)) return JINF_HIP_ERR_INVALID;
    if (cols % 256 != 0 || cols > kMvMaxTiles * kMvTile * 32 || !aligned(w, 16) ||
        !aligned(x, 16)) {
        const int64_t grid = ((int64_t)rows + kMvWaves - 1) / kMvWaves;
        return launch(matvec_q4_0_any_kernel, dim3((unsigned)grid), dim3(kMvWaves * kWave), 0,
                      stream, static_cast<const uint8_t*>(w), (int64_t)(cols / 32) * 18, x, y,
                      rows, cols / 32);
    }
    // Two rows per item; 512 workgroups (two per CU on 256 CUs) measured best
    // for 4096-14336 rows; each wave then streams several items.
    return mv_launch<2>(w, x, y, rows, cols, 512, stream);
}

}  // namespace jinf

extern "C" int jinf_matvec_q4_0(const void* weight, const float* x, float* y, int rows,
                                int cols, hipStream_t stream) {
    return jinf::matvec_q4_0(weight, x, y, rows, cols, stream);
}

// Drop-in for cuda/matmul_kernels.cu:198-225.  Q4_0 (qtype 2) is served here;
// other qtypes are reported on stderr like the reference's default branch.
extern "C" void jinf_cuda_dequant_matvec(const void* weight, const float* input, float* output,
                                         int rows, int cols, int qtype, hipStream_t stream) {
    if (rows == 0 || cols == 0) return;
    if (qtype != 2) {
        JINF_LOG("Unsupported qtype %d for dequant_matvec", qtype);
        return;
    }
    if (jinf::matvec_q4_0(weight, input, output, rows, cols, stream) == JINF_HIP_ERR_INVALID)
        JINF_LOG("jinf_cuda_dequant_matvec: invalid argument (rows=%d cols=%d)", rows, cols);
}
