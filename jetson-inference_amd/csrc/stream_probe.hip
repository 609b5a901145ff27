// Bandwidth probes: the achievable HBM rate of each hot-path kernel's traffic
// pattern on this GPU, measured with kernels that move the same bytes in the
// same launch geometry and do no arithmetic.  bench.py times each kernel next
// to its probe and reports the kernel's fraction of that ceiling beside its
// fraction of the 8 TB/s peak.  No counterpart in the reference.
//
// Every probe moves 16-byte units with nontemporal loads and stores, like the
// kernels, U = 1, 2 or 4 units per lane with all loads issued before any
// store.  With the exchange option each wave exchanges one word across lanes
// before storing (a cross-lane permute of the xor of its loads), so every
// store of a wave waits for all of the wave's loads, as the kernels' stores
// wait for their reductions or their (cos, sin) permutes; without it each
// lane's stores wait only for its own loads.  Which is faster depends on the
// pattern: an in-place copy at the RoPE config-2 shape took 3.00 us with the
// exchange and 3.98 us without, so bench.py times every variant and takes the
// fastest.  The stored data is the loaded data with its lowest bit flipped by
// the exchanged word; the contents are meaningless.
#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/probe_hip.h"

namespace jinf {

// xor of the lane's loaded words, permuted from the next lane of the wave.
__device__ __forceinline__ uint32_t wave_token(uint32_t acc) {
    return (uint32_t)__shfl((int)acc, (int)((threadIdx.x + 1) & (kWave - 1)), kWave) & 1u;
}

// RoPE geometry: grid (rows, ceil((ua + ub) / (128 U))), 128 lanes; unit u
// of a row is unit u of a's row (u < ua) or unit u - ua of b's row; lane l of
// tile y owns units y * 128 U + l + 128 j, j < U; in place.
constexpr int kProbeRowsBlock = 128;

template <int U, bool X>
__global__ __launch_bounds__(kProbeRowsBlock) void probe_rows_inplace_kernel(
    uint8_t* a, int64_t ld_a, int ua, uint8_t* b, int64_t ld_b, int ub) {
    const int64_t t = blockIdx.x;
    uint8_t* p[U];
    uint4 v[U];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int u = blockIdx.y * kProbeRowsBlock * U + threadIdx.x + kProbeRowsBlock * j;
        p[j] = nullptr;
        v[j] = make_uint4(0, 0, 0, 0);
        if (u < ua + ub) {
            p[j] = u < ua ? a + t * ld_a + (int64_t)u * 16 : b + t * ld_b + (int64_t)(u - ua) * 16;
            v[j] = ld16<true>(p[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) acc ^= v[j].x ^ v[j].w;
    const uint32_t z = X ? wave_token(acc) : (acc & 1u);
#pragma unroll
    for (int j = 0; j < U; ++j) {
        if (p[j]) {
            v[j].x ^= z;
            st16<true>(p[j], v[j]);
        }
    }
}

// Flat streams: unit i of every input is read and unit i of every output is
// written by the same lane; 256 lanes, U units each (i = block * 256 U +
// lane + 256 j).
constexpr int kProbeStreamBlock = 256;

template <int U, bool X>
__global__ __launch_bounds__(kProbeStreamBlock) void probe_stream_kernel(
    uint8_t* out0, uint8_t* out1, const uint8_t* in0, const uint8_t* in1, int64_t n_units) {
    const int64_t i0 = (int64_t)blockIdx.x * kProbeStreamBlock * U + threadIdx.x;
    uint4 v0[U], v1[U];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int64_t i = i0 + (int64_t)kProbeStreamBlock * j;
        v0[j] = make_uint4(0, 0, 0, 0);
        v1[j] = make_uint4(0, 0, 0, 0);
        if (i < n_units) {
            v0[j] = ld16<true>(in0 + i * 16);
            if (in1) v1[j] = ld16<true>(in1 + i * 16);
        }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) acc ^= v0[j].y ^ v1[j].z;
    const uint32_t z = X ? wave_token(acc) : (acc & 1u);
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int64_t i = i0 + (int64_t)kProbeStreamBlock * j;
        if (i < n_units) {
            v0[j].x ^= z;
            v1[j].x ^= z;
            st16<true>(out0 + i * 16, v0[j]);
            if (out1) st16<true>(out1 + i * 16, v1[j]);
        }
    }
}

// Flat streams in any of several launch layouts (the geometry-free curve):
// BS lanes of U units per workgroup, either one pass over a grid that covers
// the units or a grid-stride loop over a capped number of workgroups.  Unit i
// of every input is read and unit i of every output written by one lane.
// Store order XM: 0, every store after all of the lane's loads; 1, every
// store after a cross-lane exchange; 2, the first output's unit stored as
// soon as that unit's loads are in (from them alone), the second output
// after a cross-lane exchange (a row norm's order: r' before the reduction,
// y after it).
template <int U, int XM, int BS>
__global__ __launch_bounds__(BS) void probe_flat_kernel(uint8_t* out0, uint8_t* out1,
                                                       const uint8_t* in0, const uint8_t* in1,
                                                       int64_t n_units) {
    constexpr bool X = XM != 0;
    const int64_t step = (int64_t)gridDim.x * BS * U;
    for (int64_t i0 = (int64_t)blockIdx.x * BS * U + threadIdx.x; i0 - threadIdx.x < n_units;
         i0 += step) {
        uint4 v0[U], v1[U];
        uint32_t acc = 0;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t i = i0 + (int64_t)BS * j;
            v0[j] = make_uint4(0, 0, 0, 0);
            v1[j] = make_uint4(0, 0, 0, 0);
            if (i < n_units) {
                v0[j] = ld16<true>(in0 + i * 16);
                if (in1) v1[j] = ld16<true>(in1 + i * 16);
            }
        }
        if constexpr (XM == 2) {
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int64_t i = i0 + (int64_t)BS * j;
                if (i < n_units) {
                    uint4 o = v0[j];
                    o.x ^= v1[j].z & 1u;
                    st16<true>(out0 + i * 16, o);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < U; ++j) acc ^= v0[j].y ^ v1[j].z;
        const uint32_t z = X ? wave_token(acc) : (acc & 1u);
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t i = i0 + (int64_t)BS * j;
            if (i < n_units) {
                v0[j].x ^= z;
                v1[j].x ^= z;
                if constexpr (XM != 2) st16<true>(out0 + i * 16, v0[j]);
                if (out1) st16<true>(out1 + i * 16, v1[j]);
            }
        }
    }
}

// Read-only streams (a GEMV's weight traffic) in the layouts above: every
// unit of `in` is read once; the xor of a workgroup's loads is stored to
// sink[0] only when it equals a value no input of the probe produces, so the
// loads cannot be dropped and nothing is written in practice.
template <int U, int BS>
__global__ __launch_bounds__(BS) void probe_read_kernel(const uint8_t* in, int64_t n_units,
                                                       uint32_t* sink) {
    const int64_t step = (int64_t)gridDim.x * BS * U;
    uint32_t acc = 0;
    for (int64_t i0 = (int64_t)blockIdx.x * BS * U + threadIdx.x; i0 - threadIdx.x < n_units;
         i0 += step) {
        uint4 v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t i = i0 + (int64_t)BS * j;
            v[j] = make_uint4(0, 0, 0, 0);
            if (i < n_units) v[j] = ld16<true>(in + i * 16);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (acc == 0x7F3A1C5Du) sink[0] = acc;
}

// Gather geometry: grid (ids, ceil(out_units / (256 U))), 256 lanes of U
// output units; output unit u of row r is written from unit about
// u * in_units / out_units of table row ids[r] (in_units <= out_units), so
// neighbouring lanes share input units the way the Q4_0 gather's lanes share
// their blocks.  An id outside [0, n_table_rows) reads nothing.
constexpr int kProbeGatherBlock = 256;

template <int U, bool X>
__global__ __launch_bounds__(kProbeGatherBlock) void probe_gather_kernel(
    uint8_t* out, int64_t ld_out, int out_units, const uint8_t* table, int64_t ld_table,
    int in_units, const int32_t* ids, int n_table_rows) {
    const int64_t r = blockIdx.x;
    const int64_t id = ids ? ids[r] : r;
    const bool ok = id >= 0 && id < n_table_rows;
    // input unit of output unit u: floor(u * in / out) through an fp32 ratio
    // (no integer division per lane), clamped to the row
    const float ratio = (float)in_units / (float)out_units;
    uint4 v[U];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int u = blockIdx.y * kProbeGatherBlock * U + threadIdx.x + kProbeGatherBlock * j;
        v[j] = make_uint4(0, 0, 0, 0);
        if (u < out_units && ok) {
            int iu = (int)((float)u * ratio);
            iu = iu < in_units ? iu : in_units - 1;
            // cached load, as the gather reads its blocks: neighbouring
            // waves share table lines
            v[j] = ld16<false>(table + id * ld_table + (int64_t)iu * 16);
        }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) acc ^= v[j].x ^ v[j].z;
    const uint32_t z = X ? wave_token(acc) : (acc & 1u);
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int u = blockIdx.y * kProbeGatherBlock * U + threadIdx.x + kProbeGatherBlock * j;
        if (u < out_units) {
            v[j].x ^= z;
            st16<true>(out + r * ld_out + (int64_t)u * 16, v[j]);
        }
    }
}

// Masked-softmax geometry: grid (rows_per_len, length entries), BS lanes of
// 4 units each per row; row r = y * rows_per_len + x has lens[y] live floats
// (clamped to [0, n_cols]); only its whole 16-byte units are moved.
template <int BS>
__global__ __launch_bounds__(BS) void probe_rows_ragged_kernel(
    uint8_t* out, int64_t ld_out, const uint8_t* in, int64_t ld_in, int n_cols,
    const int32_t* lens, int rows_per_len, int n_rows) {
    constexpr int C = 4;
    const int64_t row = (int64_t)blockIdx.y * rows_per_len + blockIdx.x;
    int L = row < n_rows ? (lens ? lens[blockIdx.y] : n_cols) : 0;
    L = L < 0 ? 0 : (L > n_cols ? n_cols : L);
    const int nfull = L >> 2;
    const uint8_t* x = in + row * ld_in;
    uint8_t* y = out + row * ld_out;
    uint4 v[C];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const int c = threadIdx.x + j * BS;
        v[j] = make_uint4(0, 0, 0, 0);
        if (c < nfull) v[j] = ld16<true>(x + (int64_t)c * 16);
    }
#pragma unroll
    for (int j = 0; j < C; ++j) acc ^= v[j].y;
    const uint32_t z = wave_token(acc);
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const int c = threadIdx.x + j * BS;
        if (c < nfull) {
            v[j].x ^= z;
            st16<true>(y + (int64_t)c * 16, v[j]);
        }
    }
}

static bool al16(const void* p) { return aligned(p, 16); }

}  // namespace jinf

extern "C" int jinf_probe_rows_inplace(void* a, int64_t ld_a, int units_a, void* b,
                                       int64_t ld_b, int units_b, int n_rows,
                                       int units_per_lane, int exchange, hipStream_t stream) {
    using namespace jinf;
    const int U = units_per_lane;
    if (n_rows < 0 || units_a < 0 || units_b < 0 || (U != 1 && U != 2 && U != 4))
        return JINF_HIP_ERR_INVALID;
    if (n_rows == 0 || units_a + units_b == 0) return JINF_HIP_OK;
    if ((units_a && (!a || !al16(a) || ld_a % 16 || ld_a < (int64_t)units_a * 16)) ||
        (units_b && (!b || !al16(b) || ld_b % 16 || ld_b < (int64_t)units_b * 16)))
        return JINF_HIP_ERR_INVALID;
    const int64_t gy = ((int64_t)units_a + units_b + kProbeRowsBlock * U - 1) /
                       (kProbeRowsBlock * U);
    if (gy > 65535) return JINF_HIP_ERR_INVALID;
    auto go = [&](auto kern) {
        return launch(kern, dim3(n_rows, (unsigned)gy), dim3(kProbeRowsBlock), 0, stream,
                      static_cast<uint8_t*>(a), ld_a, units_a, static_cast<uint8_t*>(b), ld_b,
                      units_b);
    };
    if (exchange)
        return U == 1 ? go(probe_rows_inplace_kernel<1, true>)
                      : U == 2 ? go(probe_rows_inplace_kernel<2, true>)
                               : go(probe_rows_inplace_kernel<4, true>);
    return U == 1 ? go(probe_rows_inplace_kernel<1, false>)
                  : U == 2 ? go(probe_rows_inplace_kernel<2, false>)
                           : go(probe_rows_inplace_kernel<4, false>);
}

extern "C" int jinf_probe_stream(void* out0, void* out1, const void* in0, const void* in1,
                                 int64_t n_units, int units_per_lane, int exchange,
                                 hipStream_t stream) {
    using namespace jinf;
    const int U = units_per_lane;
    if (n_units < 0 || (U != 1 && U != 2 && U != 4)) return JINF_HIP_ERR_INVALID;
    if (n_units == 0) return JINF_HIP_OK;
    if (!out0 || !in0 || !al16(out0) || !al16(in0) || (out1 && !al16(out1)) ||
        (in1 && !al16(in1)))
        return JINF_HIP_ERR_INVALID;
    const int64_t gx = (n_units + kProbeStreamBlock * U - 1) / (kProbeStreamBlock * U);
    if (gx > 0x7FFFFFFF) return JINF_HIP_ERR_INVALID;
    auto go = [&](auto kern) {
        return launch(kern, dim3((unsigned)gx), dim3(kProbeStreamBlock), 0, stream,
                      static_cast<uint8_t*>(out0), static_cast<uint8_t*>(out1),
                      static_cast<const uint8_t*>(in0), static_cast<const uint8_t*>(in1),
                      n_units);
    };
    if (exchange)
        return U == 1 ? go(probe_stream_kernel<1, true>)
                      : U == 2 ? go(probe_stream_kernel<2, true>) : go(probe_stream_kernel<4, true>);
    return U == 1 ? go(probe_stream_kernel<1, false>)
                  : U == 2 ? go(probe_stream_kernel<2, false>) : go(probe_stream_kernel<4, false>);
}

extern "C" int jinf_probe_stream_layout(void* out0, void* out1, const void* in0,
                                        const void* in1, int64_t n_units, int units_per_lane,
                                        int exchange, int block_lanes, int max_groups,
                                        hipStream_t stream) {
    using namespace jinf;
    const int U = units_per_lane;
    const int B = block_lanes;
    if (n_units < 0 || (U != 1 && U != 2 && U != 4) || max_groups < 0 ||
        (B != 64 && B != 128 && B != 256 && B != 512 && B != 1024) || exchange < 0 ||
        exchange > 2)
        return JINF_HIP_ERR_INVALID;
    if (n_units == 0) return JINF_HIP_OK;
    if (!out0 || !in0 || !al16(out0) || !al16(in0) || (out1 && !al16(out1)) ||
        (in1 && !al16(in1)))
        return JINF_HIP_ERR_INVALID;
    int64_t gx = (n_units + (int64_t)B * U - 1) / ((int64_t)B * U);
    if (max_groups > 0 && gx > max_groups) gx = max_groups;
    if (gx > 0x7FFFFFFF) return JINF_HIP_ERR_INVALID;
    auto go = [&](auto kern) {
        return launch(kern, dim3((unsigned)gx), dim3(B), 0, stream, static_cast<uint8_t*>(out0),
                      static_cast<uint8_t*>(out1), static_cast<const uint8_t*>(in0),
                      static_cast<const uint8_t*>(in1), n_units);
    };
#define JINF_PROBE_FLAT_X(XM, BS)                                                           \
    (U == 1 ? go(probe_flat_kernel<1, XM, BS>)                                              \
            : U == 2 ? go(probe_flat_kernel<2, XM, BS>) : go(probe_flat_kernel<4, XM, BS>))
#define JINF_PROBE_FLAT(BS)                                                                 \
    (exchange == 2 ? JINF_PROBE_FLAT_X(2, BS)                                               \
                   : exchange ? JINF_PROBE_FLAT_X(1, BS) : JINF_PROBE_FLAT_X(0, BS))
    switch (B) {
        case 64: return JINF_PROBE_FLAT(64);
        case 128: return JINF_PROBE_FLAT(128);
        case 256: return JINF_PROBE_FLAT(256);
        case 512: return JINF_PROBE_FLAT(512);
        default: return JINF_PROBE_FLAT(1024);
    }
#undef JINF_PROBE_FLAT
#undef JINF_PROBE_FLAT_X
}

extern "C" int jinf_probe_read_layout(const void* in, int64_t n_units, void* sink,
                                      int units_per_lane, int block_lanes, int max_groups,
                                      hipStream_t stream) {
    using namespace jinf;
    const int U = units_per_lane;
    const int B = block_lanes;
    if (n_units < 0 || (U != 1 && U != 2 && U != 4) || max_groups < 0 ||
        (B != 64 && B != 128 && B != 256 && B != 512 && B != 1024))
        return JINF_HIP_ERR_INVALID;
    if (n_units == 0) return JINF_HIP_OK;
    if (!in || !sink || !al16(in) || !aligned(sink, 4)) return JINF_HIP_ERR_INVALID;
    int64_t gx = (n_units + (int64_t)B * U - 1) / ((int64_t)B * U);
    if (max_groups > 0 && gx > max_groups) gx = max_groups;
    if (gx > 0x7FFFFFFF) return JINF_HIP_ERR_INVALID;
    auto go = [&](auto kern) {
        return launch(kern, dim3((unsigned)gx), dim3(B), 0, stream,
                      static_cast<const uint8_t*>(in), n_units, static_cast<uint32_t*>(sink));
    };
#define JINF_PROBE_READ(BS)                                                                  \
    (U == 1 ? go(probe_read_kernel<1, BS>)                                                   \
            : U == 2 ? go(probe_read_kernel<2, BS>) : go(probe_read_kernel<4, BS>))
    switch (B) {
        case 64: return JINF_PROBE_READ(64);
        case 128: return JINF_PROBE_READ(128);
        case 256: return JINF_PROBE_READ(256);
        case 512: return JINF_PROBE_READ(512);
        default: return JINF_PROBE_READ(1024);
    }
#undef JINF_PROBE_READ
}

extern "C" int jinf_probe_gather(void* out, int64_t ld_out, int out_units, const void* table,
                                 int64_t ld_table, int in_units, int n_table_rows,
                                 const int32_t* ids, int n_ids, int units_per_lane,
                                 int exchange, hipStream_t stream) {
    using namespace jinf;
    const int U = units_per_lane;
    if (n_ids < 0 || out_units < 0 || in_units < 0 || in_units > out_units ||
        (U != 1 && U != 2 && U != 4))
        return JINF_HIP_ERR_INVALID;
    if (n_ids == 0 || out_units == 0) return JINF_HIP_OK;
    if (in_units == 0 || n_table_rows <= 0 || (!ids && n_ids > n_table_rows))
        return JINF_HIP_ERR_INVALID;
    if (!out || !table || !al16(out) || !al16(table) || ld_out % 16 || ld_table % 16 ||
        ld_out < (int64_t)out_units * 16 || ld_table < (int64_t)in_units * 16)
        return JINF_HIP_ERR_INVALID;
    const int64_t gy = ((int64_t)out_units + kProbeGatherBlock * U - 1) / (kProbeGatherBlock * U);
    if (gy > 65535) return JINF_HIP_ERR_INVALID;
    auto go = [&](auto kern) {
        return launch(kern, dim3(n_ids, (unsigned)gy), dim3(kProbeGatherBlock), 0, stream,
                      static_cast<uint8_t*>(out), ld_out, out_units,
                      static_cast<const uint8_t*>(table), ld_table, in_units, ids, n_table_rows);
    };
    if (exchange)
        return U == 1 ? go(probe_gather_kernel<1, true>)
                      : U == 2 ? go(probe_gather_kernel<2, true>) : go(probe_gather_kernel<4, true>);
    return U == 1 ? go(probe_gather_kernel<1, false>)
                  : U == 2 ? go(probe_gather_kernel<2, false>) : go(probe_gather_kernel<4, false>);
}

extern "C" int jinf_probe_rows_ragged(void* out, int64_t ld_out, const void* in, int64_t ld_in,
                                      int n_cols, const int32_t* lens, int rows_per_len,
                                      int n_rows, hipStream_t stream) {
    using namespace jinf;
    if (n_rows < 0 || n_cols < 0 || (lens && rows_per_len <= 0)) return JINF_HIP_ERR_INVALID;
    if (n_rows == 0 || n_cols == 0) return JINF_HIP_OK;
    if (!out || !in || !al16(out) || !al16(in) || ld_out % 16 || ld_in % 16 ||
        ld_out < (int64_t)n_cols * 4 || ld_in < (int64_t)n_cols * 4 || n_cols > 16384)
        return JINF_HIP_ERR_INVALID;
    const int rpl = lens ? rows_per_len : n_rows;
    const int64_t groups = ((int64_t)n_rows + rpl - 1) / rpl;
    if (groups > 65535) return JINF_HIP_ERR_INVALID;
    const dim3 grid((unsigned)(rpl < n_rows ? rpl : n_rows), (unsigned)groups);
    auto go = [&](auto kern, int bs) {
        return launch(kern, grid, dim3(bs), 0, stream, static_cast<uint8_t*>(out), ld_out,
                      static_cast<const uint8_t*>(in), ld_in, n_cols, lens, rpl, n_rows);
    };
    // lanes as the softmax picks them: 4 units per lane
    if (n_cols <= 256) return go(probe_rows_ragged_kernel<64>, 64);
    if (n_cols <= 4096) return go(probe_rows_ragged_kernel<256>, 256);
    if (n_cols <= 8192) return go(probe_rows_ragged_kernel<512>, 512);
    return go(probe_rows_ragged_kernel<1024>, 1024);
}
