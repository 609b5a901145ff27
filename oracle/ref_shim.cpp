// Exposes the reference's own CPU routines (compiled from
// /root/reference/src/quant.cpp where it lies) under C names, so the oracle's
// restatement can be checked against them.  Test infrastructure only.
#include "jinf/quant.h"

extern "C" void jref_dequantize_q4_0(const void* blocks, float* out, int n_blocks) {
    jinf_dequantize_q4_0(static_cast<const jinf_block_q4_0*>(blocks), out, n_blocks);
}

// The reference's fp16 -> fp32 conversion, reached through its generic
// dispatcher (src/quant.cpp:108-136, JINF_TYPE_F16 branch).
extern "C" void jref_f16_to_f32(const void* halfs, float* out, long long n) {
    jinf_dequantize(halfs, JINF_TYPE_F16, out, (int64_t)n);
}

extern "C" void jref_dequantize_q4_K(const void* blocks, float* out, int n_blocks) {
    jinf_dequantize_q4_K(static_cast<const jinf_block_q4_K*>(blocks), out, n_blocks);
}

extern "C" void jref_dequantize_q8_0(const void* blocks, float* out, int n_blocks) {
    jinf_dequantize_q8_0(static_cast<const jinf_block_q8_0*>(blocks), out, n_blocks);
}

// The reference's GGUF reader (src/gguf.cpp, compiled where it lies): a text
// dump of everything it parsed, one field per line, in the format the tests
// build from this repository's reader.  Returns the jinf_status of the open;
// the dump is truncated to cap bytes.
#include "jinf/gguf.h"
#include <cstdio>
#include <cstring>
#include <string>

static void dump_kv(std::string& s, const jinf_gguf_kv* kv) {
    char b[256];
    s += "kv ";
    s += kv->key;
    snprintf(b, sizeof b, " %d ", (int)kv->type);
    s += b;
    switch (kv->type) {
        case JINF_GGUF_TYPE_UINT8: snprintf(b, sizeof b, "%u", (unsigned)kv->val_u8); break;
        case JINF_GGUF_TYPE_INT8: snprintf(b, sizeof b, "%d", (int)kv->val_i8); break;
        case JINF_GGUF_TYPE_UINT16: snprintf(b, sizeof b, "%u", (unsigned)kv->val_u16); break;
        case JINF_GGUF_TYPE_INT16: snprintf(b, sizeof b, "%d", (int)kv->val_i16); break;
        case JINF_GGUF_TYPE_UINT32: snprintf(b, sizeof b, "%u", kv->val_u32); break;
        case JINF_GGUF_TYPE_INT32: snprintf(b, sizeof b, "%d", kv->val_i32); break;
        case JINF_GGUF_TYPE_FLOAT32: snprintf(b, sizeof b, "%.9g", (double)kv->val_f32); break;
        case JINF_GGUF_TYPE_BOOL: snprintf(b, sizeof b, "%d", kv->val_bool ? 1 : 0); break;
        case JINF_GGUF_TYPE_UINT64: snprintf(b, sizeof b, "%llu", (unsigned long long)kv->val_u64); break;
        case JINF_GGUF_TYPE_INT64: snprintf(b, sizeof b, "%lld", (long long)kv->val_i64); break;
        case JINF_GGUF_TYPE_FLOAT64: snprintf(b, sizeof b, "%.17g", kv->val_f64); break;
        case JINF_GGUF_TYPE_STRING: s += kv->val_str.data; b[0] = 0; break;
        case JINF_GGUF_TYPE_ARRAY:
            snprintf(b, sizeof b, "[%d x %llu]", (int)kv->val_arr.elem_type,
                     (unsigned long long)kv->val_arr.count);
            break;
        default: b[0] = 0; break;
    }
    s += b;
    s += "\n";
}

extern "C" int jref_gguf_dump(const char* path, char* out, int cap) {
    jinf_gguf_file* f = nullptr;
    const jinf_status st = jinf_gguf_open(&f, path);
    std::string s;
    if (st == JINF_OK) {
        char b[512];
        snprintf(b, sizeof b, "version %u\nalignment %u\ndata_offset %zu\nkv_count %llu\ntensor_count %llu\n",
                 f->version, f->alignment, f->data_offset, (unsigned long long)f->kv_count,
                 (unsigned long long)f->tensor_count);
        s += b;
        for (uint64_t i = 0; i < f->kv_count; ++i) dump_kv(s, &f->kvs[i]);
        for (uint64_t i = 0; i < f->tensor_count; ++i) {
            const jinf_gguf_tensor_info* t = &f->tensor_infos[i];
            snprintf(b, sizeof b, "tensor %s %u", t->name, t->n_dims);
            s += b;
            for (uint32_t d = 0; d < t->n_dims; ++d) {
                snprintf(b, sizeof b, " %lld", (long long)t->shape[d]);
                s += b;
            }
            snprintf(b, sizeof b, " type %d offset %llu n_elements %lld n_bytes %zu\n", (int)t->type,
                     (unsigned long long)t->offset, (long long)t->n_elements, t->n_bytes);
            s += b;
        }
        const jinf_model_hparams& h = f->hparams;
        snprintf(b, sizeof b,
                 "hparams %s %u %u %u %u %u %u %u %.9g %.9g\n", h.arch, h.n_layers, h.n_embd,
                 h.n_heads, h.n_heads_kv, h.n_ff, h.n_vocab, h.n_ctx_train,
                 (double)h.rope_freq_base, (double)h.rms_norm_eps);
        s += b;
        jinf_gguf_close(f);
    }
    const size_t n = s.size() < (size_t)cap - 1 ? s.size() : (size_t)cap - 1;
    memcpy(out, s.data(), n);
    out[n] = 0;
    return (int)st;
}

// ---- .nvmw reader (src/nvmw.cpp) ----
// jref_nvmw_dump: open a file with the reference reader and print what it
// parsed, one item per line, in the format the tests build from this
// repository's reader.  Returns the jinf_status of the open.
#include "jinf/nvmw.h"

extern "C" int jref_nvmw_dump(const char* path, char* out, int cap) {
    jinf_nvmw_reader* r = nullptr;
    const jinf_status st = jinf_nvmw_open(&r, path);
    std::string s;
    if (st == JINF_OK) {
        char b[512];
        const jinf_nvmw_header* h = jinf_nvmw_get_header(r);
        snprintf(b, sizeof b,
                 "header %u %u %u %u %llu %llu %llu %llu %llu %llu\n"
                 "hparams %u %u %u %u %u %u %.9g %.9g %d %llu\n",
                 h->magic, h->version, h->n_layers, h->n_tensors,
                 (unsigned long long)h->index_offset, (unsigned long long)h->index_size,
                 (unsigned long long)h->hot_offset, (unsigned long long)h->hot_size,
                 (unsigned long long)h->cold_start_offset, (unsigned long long)h->cold_total_size,
                 h->n_embd, h->n_heads, h->n_heads_kv, h->n_ff, h->n_vocab, h->n_ctx_train,
                 (double)h->rope_freq_base, (double)h->rms_norm_eps, (int)h->primary_type,
                 (unsigned long long)h->bundle_index_offset);
        s += b;
        for (int L = 0; L < (int)h->n_layers; ++L) {
            uint64_t off = 0, size = 0;
            jinf_nvmw_get_layer_cold_range(r, L, &off, &size);
            snprintf(b, sizeof b, "layer %d %llu %llu\n", L, (unsigned long long)off,
                     (unsigned long long)size);
            s += b;
        }
        int n = 0;
        const jinf_nvmw_tensor_entry* te = jinf_nvmw_get_tensor_entries(r, &n);
        for (int i = 0; i < n; ++i) {
            const jinf_nvmw_tensor_entry& t = te[i];
            snprintf(b, sizeof b, "tensor %s %d %lld %lld %lld %lld %u %llu %llu %d %d\n", t.name,
                     (int)t.type, (long long)t.shape[0], (long long)t.shape[1],
                     (long long)t.shape[2], (long long)t.shape[3], t.n_dims,
                     (unsigned long long)t.offset, (unsigned long long)t.n_bytes, t.layer_index,
                     (int)t.is_hot);
            s += b;
        }
        snprintf(b, sizeof b, "bundles %d\n", jinf_nvmw_has_bundles(r) ? 1 : 0);
        s += b;
        jinf_nvmw_close(r);
    }
    const size_t n = s.size() < (size_t)cap - 1 ? s.size() : (size_t)cap - 1;
    memcpy(out, s.data(), n);
    out[n] = 0;
    return (int)st;
}
