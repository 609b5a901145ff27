/*
 * jinf MI355X bandwidth probes: kernels that move a hot-path kernel's bytes
 * in its launch geometry and do no arithmetic, so that the time of the probe
 * is the achievable time of that traffic pattern on the GPU (the "ceiling"
 * bench.py reports each kernel against).  No counterpart in the reference.
 *
 * All pointers are device pointers, 16-byte aligned, with row strides in
 * BYTES that are multiples of 16; units are 16 bytes.  Every probe overwrites
 * its outputs with its inputs' bytes, one bit flipped (meaningless data).
 * units_per_lane (1, 2 or 4) sets how many units each lane moves per array,
 * all loads issued before any store; exchange != 0 makes every store of a
 * wave wait for all of the wave's loads (one cross-lane permute), exchange 0
 * lets each lane store after its own loads (jinf_probe_stream_layout's
 * exchange 2: the first output after its own loads, the second after the
 * permute).  bench.py takes the fastest
 * variant as a kernel's ceiling.  Work is asynchronous on `stream`; nothing
 * allocates.  Return 0, or 5 for an invalid argument (nothing enqueued), or
 * 3 if the launch failed.
 *
 * This header includes no HIP or CUDA header.
 */
#ifndef JINF_PROBE_HIP_H
#define JINF_PROBE_HIP_H

#include <stdint.h>
#include "kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* In place, RoPE's geometry (jinf_rope_rows): n_rows rows, each units_a units
 * of a (stride ld_a) then units_b units of b (stride ld_b); 128-lane
 * workgroups. */
int jinf_probe_rows_inplace(void* a, int64_t ld_a, int units_a, void* b, int64_t ld_b,
                            int units_b, int n_rows, int units_per_lane, int exchange,
                            hipStream_t stream);

/* Flat streams (SwiGLU, residual add, residual + RMSNorm): unit i of in0 (and
 * of in1 unless NULL) is read and unit i of out0 (and of out1 unless NULL)
 * written, i < n_units; 256-lane workgroups.  out0 may equal in0. */
int jinf_probe_stream(void* out0, void* out1, const void* in0, const void* in1,
                      int64_t n_units, int units_per_lane, int exchange, hipStream_t stream);

/* Flat streams as jinf_probe_stream, in a chosen launch layout (for the
 * geometry-free bandwidth curve): block_lanes (64, 128, 256, 512 or 1024)
 * lanes of units_per_lane units per workgroup; max_groups 0 launches one pass
 * over enough workgroups to cover n_units, max_groups > 0 caps the grid at
 * that many workgroups, which loop over the units with a grid stride.
 * exchange: 0, stores after all of a lane's loads; 1, stores after a
 * cross-lane exchange; 2, out0's units stored straight after their own loads
 * and out1's after a cross-lane exchange. */
int jinf_probe_stream_layout(void* out0, void* out1, const void* in0, const void* in1,
                             int64_t n_units, int units_per_lane, int exchange,
                             int block_lanes, int max_groups, hipStream_t stream);

/* A read-only stream (a GEMV's weight traffic) in the layouts of
 * jinf_probe_stream_layout: n_units 16-byte units of `in` read once; sink (4
 * bytes) is written only if the loaded words xor to one fixed value, which no
 * probe input produces, so in practice nothing is written. */
int jinf_probe_read_layout(const void* in, int64_t n_units, void* sink, int units_per_lane,
                           int block_lanes, int max_groups, hipStream_t stream);

/* Row gather (the Q4_0 embedding gather's geometry): output row r
 * (ld_out bytes apart, out_units units) is written from table row ids[r]
 * (row r when ids is NULL; ld_table bytes apart, in_units <= out_units units,
 * each read by the lanes whose output it feeds).  An id outside
 * [0, n_table_rows) reads nothing. */
int jinf_probe_gather(void* out, int64_t ld_out, int out_units, const void* table,
                      int64_t ld_table, int in_units, int n_table_rows, const int32_t* ids,
                      int n_ids, int units_per_lane, int exchange, hipStream_t stream);

/* Ragged fp32 rows (jinf_softmax_rows_f32's geometry, 4 units per lane): row
 * r moves its first 4 * floor(L / 4) floats, L = lens[r / rows_per_len]
 * clamped to [0, n_cols] (n_cols when lens is NULL), n_cols <= 16384. */
int jinf_probe_rows_ragged(void* out, int64_t ld_out, const void* in, int64_t ld_in,
                           int n_cols, const int32_t* lens, int rows_per_len, int n_rows,
                           hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JINF_PROBE_HIP_H */
