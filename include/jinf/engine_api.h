/* jinf's engine API under the reference's own names, for callers written
 * against it (e.g. the reference's bench/inference_bench.cpp:53-140): the
 * same entry points, argument meanings and struct layouts as
 * include/jinf/engine.h:12-47 and :159-176 of the reference, over the
 * resident-weight engine of engine_hip.h.  Linkage differs: the reference
 * declares these functions with C++ linkage (mangled names), this library
 * exports them extern "C", so a caller compiles against this header or a
 * stand-in engine.h that declares the same prototypes inside extern "C",
 * not against the reference's engine.h unchanged.  Status returns are the
 * reference's jinf_status values (an int-sized enum there, int here), 0 OK,
 * 1 I/O, 2 parse, 3 device, 4 out of memory, 5 invalid.
 *
 * config->model_path names a .nvmw file (as in the reference); every tensor is
 * uploaded into device memory, so the streaming settings (gpu_memory_budget,
 * buffer_capacity, io_queue_depth) have no role and are not read.  The KV
 * cache is fp32, the reference's.  A sparse-FFN predictor (predictor_path)
 * is not supported: create returns 5 for one. */
#ifndef JINF_ENGINE_API_H
#define JINF_ENGINE_API_H

#include <stddef.h>
#include <stdint.h>

#include "engine_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct jinf_engine jinf_engine;  /* opaque */

/* include/jinf/engine.h:25-35 of the reference, field for field */
typedef struct jinf_engine_config {
    const char* model_path;
    size_t gpu_memory_budget;
    size_t buffer_capacity;
    int max_context;
    int io_queue_depth;
    const char* predictor_path;
    float sparsity_threshold;
} jinf_engine_config;

/* the reference's defaults (include/jinf/engine.h:37-47) */
static inline jinf_engine_config jinf_engine_config_default(void) {
    jinf_engine_config c;
    c.model_path = NULL;
    c.gpu_memory_budget = (size_t)4500 * 1024 * 1024;
    c.buffer_capacity = (size_t)128 * 1024 * 1024;
    c.max_context = 512;
    c.io_queue_depth = 64;
    c.predictor_path = NULL;
    c.sparsity_threshold = 0.5f;
    return c;
}

/* the reference's jinf_perf_stats (include/jinf/engine.h:14-22) */
typedef jinf_hip_perf_stats jinf_perf_stats;

/* jinf_engine_create (src/engine.cpp:40-188): loads the .nvmw file and
 * builds the engine. */
int jinf_engine_create(jinf_engine** e, const jinf_engine_config* config);

/* jinf_engine_destroy */
void jinf_engine_destroy(jinf_engine* e);

/* jinf_engine_forward (src/engine.cpp:684-760): decodes the tokens one at a
 * time and returns the device address of the last token's logits. */
int jinf_engine_forward(jinf_engine* e, const int32_t* tokens, int n_tokens, float** logits);

/* jinf_engine_generate (src/engine.cpp:762-805): greedy generation, stops
 * after token 2. */
int jinf_engine_generate(jinf_engine* e, const int32_t* prompt, int n_prompt, int32_t* output,
                         int max_tokens, int* n_generated);

/* jinf_engine_reset (src/engine.cpp:293-302): clears the KV cache, the
 * position and the counters. */
void jinf_engine_reset(jinf_engine* e);

/* jinf_engine_get_stats (src/engine.cpp:304-306) */
const jinf_perf_stats* jinf_engine_get_stats(const jinf_engine* e);

#ifdef __cplusplus
}
#endif

#endif
