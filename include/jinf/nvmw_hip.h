/*
 * jinf MI355X: .nvmw model files -- the container jinf's prepare_model tool
 * writes from a GGUF file and jinf's engine loads (reference
 * include/jinf/nvmw.h:8-157, reader src/nvmw.cpp:182-341).
 *
 * Layout (little-endian): a 4096-byte header (magic "NVMW", version, counts,
 * region offsets, model hyper-parameters), at index_offset n_layers layer
 * descriptors (absolute offset and size of each layer's cold region) and
 * n_tensors 200-byte tensor entries (GGUF name, jinf_qtype, shape, offset
 * within its region, size, layer index, hot flag), then the hot region and
 * the per-layer cold regions.  A hot tensor's bytes start at hot_offset +
 * offset, a cold one's at its layer's cold start + offset.  Version 2 files
 * may carry the sparse-FFN neuron-bundle index (bundle_index_offset != 0);
 * it is read and reported, and the engine decodes with the dense FFN.
 *
 * Parsing accepts what the reference reader accepts (it checks the magic,
 * not the version) and also rejects an index or tensor data past the end of
 * the file.  Status codes are jinf_status values (0 OK, 1 I/O, 2 parse,
 * 3 device, 4 out of memory, 5 invalid argument).  This header includes no
 * HIP or CUDA header.
 */
#ifndef JINF_NVMW_HIP_H
#define JINF_NVMW_HIP_H

#include <stdint.h>
#include "kernels_ext.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct jinf_hip_nvmw jinf_hip_nvmw;

/* The header fields (jinf_nvmw_header, include/jinf/nvmw.h:66-100). */
typedef struct jinf_hip_nvmw_header {
    uint32_t magic, version, n_layers, n_tensors;
    uint64_t index_offset, index_size, hot_offset, hot_size;
    uint64_t cold_start_offset, cold_total_size;
    uint32_t n_embd, n_heads, n_heads_kv, n_ff, n_vocab, n_ctx_train;
    float    rope_freq_base, rms_norm_eps;
    int32_t  primary_type;
    uint64_t bundle_index_offset;
} jinf_hip_nvmw_header;

/* One tensor entry (jinf_nvmw_tensor_entry, include/jinf/nvmw.h:24-34), with
 * the absolute file offset of its bytes resolved. */
typedef struct jinf_hip_nvmw_tensor {
    const char* name;
    int         qtype;
    int64_t     shape[4];
    uint32_t    n_dims;
    uint64_t    offset;        /* within its region, as stored */
    uint64_t    n_bytes;
    int32_t     layer_index;   /* -1: not a layer tensor */
    int         is_hot;
    uint64_t    file_offset;   /* absolute */
} jinf_hip_nvmw_tensor;

/* Parse a file (replaces jinf_nvmw_open, src/nvmw.cpp:194-259). */
int  jinf_hip_nvmw_load(jinf_hip_nvmw** out, const char* path);
void jinf_hip_nvmw_free(jinf_hip_nvmw* file);                      /* jinf_nvmw_close */

const jinf_hip_nvmw_header* jinf_hip_nvmw_header_of(const jinf_hip_nvmw* file);
uint64_t jinf_hip_nvmw_n_tensors(const jinf_hip_nvmw* file);
const jinf_hip_nvmw_tensor* jinf_hip_nvmw_tensor_at(const jinf_hip_nvmw* file, uint64_t i);
/* Exact name lookup (jinf_nvmw_find_tensor, src/nvmw.cpp:289-295); -1: none. */
int64_t jinf_hip_nvmw_find_tensor(const jinf_hip_nvmw* file, const char* name);
/* Layer layer's cold region (jinf_nvmw_get_layer_cold_range,
 * src/nvmw.cpp:271-279); status 5 for a layer out of range. */
int jinf_hip_nvmw_layer_cold_range(const jinf_hip_nvmw* file, int layer, uint64_t* offset,
                                   uint64_t* size);
/* 1 when the file carries the neuron-bundle index (jinf_nvmw_has_bundles,
 * src/nvmw.cpp:299-301). */
int jinf_hip_nvmw_has_bundles(const jinf_hip_nvmw* file);

/* Copy tensor i's bytes into device memory at dst (dst_bytes >= n_bytes),
 * streaming through pinned buffers on `stream`; returns after the copies. */
int jinf_hip_nvmw_upload(const jinf_hip_nvmw* file, uint64_t i, void* dst, uint64_t dst_bytes,
                         hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JINF_NVMW_HIP_H */
