/*
 * jinf MI355X: GGUF model files -- metadata, tensor upload into device
 * memory, and the Q4_0 element-order conversion for upstream-ggml files.
 *
 * Parsing follows the reference reader (src/gguf.cpp:143-311, API
 * include/jinf/gguf.h:96-113): the same file gives the same version, counts,
 * alignment, data offset, key/value pairs, tensor infos and hyper-parameters
 * (with the reference's key names and defaults).  The handle is opaque and
 * owns every string it returns; nothing here is thread-safe for one handle
 * being freed while used.  Status codes are jinf_status values: 0 OK,
 * 1 I/O, 2 parse, 3 device, 4 out of memory, 5 invalid argument.
 *
 * This header includes no HIP or CUDA header.
 */
#ifndef JINF_GGUF_HIP_H
#define JINF_GGUF_HIP_H

#include <stdint.h>
#include "kernels_ext.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct jinf_hip_gguf jinf_hip_gguf;

/* Model hyper-parameters, the fields of jinf_model_hparams
 * (include/jinf/gguf.h:64-75). */
typedef struct jinf_hip_gguf_hparams {
    char     arch[64];
    uint32_t n_layers;
    uint32_t n_embd;
    uint32_t n_heads;
    uint32_t n_heads_kv;
    uint32_t n_ff;
    uint32_t n_vocab;
    uint32_t n_ctx_train;
    float    rope_freq_base;
    float    rms_norm_eps;
} jinf_hip_gguf_hparams;

/* One tensor: the fields of jinf_gguf_tensor_info (include/jinf/gguf.h:53-61);
 * qtype is the jinf_qtype code (= ggml type code; unknown codes read as 0). */
typedef struct jinf_hip_gguf_tensor {
    const char* name;
    uint32_t    n_dims;
    int64_t     shape[4];
    int         qtype;
    uint64_t    offset;       /* within the data section */
    int64_t     n_elements;
    uint64_t    n_bytes;
} jinf_hip_gguf_tensor;

/* Parse a GGUF v2/v3 file (replaces jinf_gguf_open, src/gguf.cpp:143-311).
 * Also rejects what the reference does not check: n_dims > 4, alignment 0,
 * tensor data past the end of the file. */
int  jinf_hip_gguf_load(jinf_hip_gguf** out, const char* path);
void jinf_hip_gguf_free(jinf_hip_gguf* file);          /* jinf_gguf_close */

uint32_t jinf_hip_gguf_version(const jinf_hip_gguf* file);
uint32_t jinf_hip_gguf_alignment(const jinf_hip_gguf* file);
uint64_t jinf_hip_gguf_data_offset(const jinf_hip_gguf* file);   /* absolute */
uint64_t jinf_hip_gguf_n_kv(const jinf_hip_gguf* file);
uint64_t jinf_hip_gguf_n_tensors(const jinf_hip_gguf* file);
const jinf_hip_gguf_hparams* jinf_hip_gguf_hparams_of(const jinf_hip_gguf* file);

/* Key/value pairs by index.  kv_type: GGUF value type 0-12 (-1 bad index);
 * kv_scalar copies a scalar's bytes (1-8) to out; kv_str: string value or
 * NULL; kv_array: element type and count of an array (its data is skipped,
 * as in the reference). */
int64_t     jinf_hip_gguf_find_kv(const jinf_hip_gguf* file, const char* key);  /* -1: none */
const char* jinf_hip_gguf_kv_key(const jinf_hip_gguf* file, uint64_t i);
int         jinf_hip_gguf_kv_type(const jinf_hip_gguf* file, uint64_t i);
int         jinf_hip_gguf_kv_scalar(const jinf_hip_gguf* file, uint64_t i, void* out);
const char* jinf_hip_gguf_kv_str(const jinf_hip_gguf* file, uint64_t i);
int         jinf_hip_gguf_kv_array(const jinf_hip_gguf* file, uint64_t i, int* elem_type,
                                   uint64_t* count);

/* Typed lookups with the reference's conversions and defaults
 * (jinf_gguf_get_str / _u32 / _f32, src/gguf.cpp:343-381). */
const char* jinf_hip_gguf_get_str(const jinf_hip_gguf* file, const char* key, const char* def);
uint32_t    jinf_hip_gguf_get_u32(const jinf_hip_gguf* file, const char* key, uint32_t def);
float       jinf_hip_gguf_get_f32(const jinf_hip_gguf* file, const char* key, float def);

/* Tensors (jinf_gguf_find_tensor, src/gguf.cpp:333-341). */
int64_t jinf_hip_gguf_find_tensor(const jinf_hip_gguf* file, const char* name);  /* -1: none */
const jinf_hip_gguf_tensor* jinf_hip_gguf_tensor_at(const jinf_hip_gguf* file, uint64_t i);

/* Copy tensor i's bytes from the file into device memory at dst (dst_bytes
 * >= n_bytes), streaming through two 32 MiB pinned buffers on `stream`
 * (file reads overlap the copies).  A loader call: it allocates and frees the
 * pinned buffers and returns after the stream has finished the copies. */
int jinf_hip_gguf_upload(const jinf_hip_gguf* file, uint64_t i, void* dst, uint64_t dst_bytes,
                         hipStream_t stream);

/* Rewrite n_blocks Q4_0 blocks in device memory, in place, from upstream
 * ggml's element order (element j in the low nibble of qs[j], element j+16
 * in its high nibble) to jinf's (elements 2i, 2i+1 in the low and high
 * nibble of qs[i]; src/quant.cpp:53-57), so that GGUF files written by
 * upstream tools decode correctly with every Q4_0 kernel here.  Blocks may
 * have any byte alignment.  No counterpart in the reference, which reads
 * upstream files in its own order. */
int jinf_hip_q4_0_repack_ggml(void* blocks, int64_t n_blocks, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JINF_GGUF_HIP_H */
