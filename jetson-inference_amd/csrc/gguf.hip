// GGUF model files: metadata parse, tensor upload into HBM, and the Q4_0
// element-order conversion for files written by upstream ggml.
//
// Parse semantics follow the reference reader (src/gguf.cpp:143-311) so the
// same file yields the same fields:
//   - magic "GGUF", version 2 or 3; tensor and key/value counts (u64);
//   - key/value pairs: string keys (at most 1 MiB, as the reference), scalar
//     types 0-12, arrays skipped element by element (their type and count are
//     kept); "general.alignment" (u32) overrides the default 32;
//   - tensor infos: name, n_dims, dims (i64), ggml type (unknown codes read as
//     F32, as the reference does), offset within the data section; the byte
//     count is ceil(n_elements / block) * block bytes (include/jinf/quant.h);
//   - the data section starts at the next multiple of the alignment;
//   - hyper-parameters from "<arch>.block_count" etc. with the reference's
//     defaults (context 2048, rope base 10000, rms eps 1e-5, kv heads = heads,
//     vocab from token_embd.weight's second dimension).
// Where the reference would fail silently or crash this reader returns a
// parse error instead: n_dims > 4 (the reference writes past shape[4]),
// alignment 0 (it divides by zero), tensor data past the end of the file.
//
// Upload streams a tensor's bytes from the file into device memory through
// two pinned staging buffers (file read of chunk k+1 overlaps the
// host-to-device copy of chunk k on the caller's stream).
//
// Element order.  jinf's Q4_0 kernels (like the reference's, quant.cpp:53-57)
// read element 2i from the low nibble of qs[i] and 2i+1 from its high nibble;
// upstream ggml stores element j in the low nibble of qs[j] and element j+16
// in its high nibble.  jinf_hip_q4_0_repack_ggml rewrites blocks written in
// the upstream order into jinf's order on the GPU, in place.
#include <errno.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <string>
#include <vector>

#include "file_io.h"
#include "jinf_device.h"
#include "jinf_host.h"
#include "jinf/gguf_hip.h"

struct jinf_hip_gguf {
    std::string path;
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    uint64_t file_size = 0;
    struct KV {
        std::string key;
        int type = 0;
        uint64_t raw = 0;       // scalar value bytes (little-endian, zero-extended)
        std::string str;        // string value
        int elem_type = -1;     // arrays
        uint64_t count = 0;
    };
    std::vector<KV> kvs;
    std::vector<std::string> names;
    std::vector<jinf_hip_gguf_tensor> tensors;
    jinf_hip_gguf_hparams hp{};
};

namespace jinf {
namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kMaxString = 1024 * 1024;

// Values per block and bytes per block of a ggml type code (quant.h:76-116).
void type_geometry(int t, int* block, int* bytes) {
    static const int blk[16] = {1, 1, 32, 32, 0, 0, 32, 32, 32, 32, 256, 256, 256, 256, 256, 256};
    static const int byt[16] = {4, 2, 18, 20, 0, 0, 22, 24, 34, 36, 84, 110, 144, 176, 210, 292};
    if (t < 0 || t > 15) {
        *block = *bytes = 0;
        return;
    }
    *block = blk[t];
    *bytes = byt[t];
}

// ggml type code -> jinf_qtype (src/gguf.cpp:117-137): the codes coincide;
// anything unknown reads as F32.
int map_type(uint32_t t) {
    switch (t) {
        case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 9:
        case 10: case 11: case 12: case 13: case 14: case 15:
            return (int)t;
        default:
            return 0;
    }
}

struct Reader {
    FILE* f;
    bool ok = true;
    template <typename T> T get() {
        T v{};
        if (ok && fread(&v, sizeof(T), 1, f) != 1) ok = false;
        return v;
    }
    bool string(std::string& s) {
        const uint64_t len = get<uint64_t>();
        if (!ok || len > kMaxString) return ok = false;
        s.resize(len);
        if (len && fread(&s[0], 1, len, f) != len) return ok = false;
        return true;
    }
    bool skip(uint64_t n) {
        if (ok && fseeko(f, (off_t)n, SEEK_CUR) != 0) ok = false;
        return ok;
    }
    // Skips one value of type t (arrays recursively).
    bool skip_value(int t, int depth = 0) {
        switch (t) {
            case 0: case 1: case 7: return skip(1);
            case 2: case 3: return skip(2);
            case 4: case 5: case 6: return skip(4);
            case 10: case 11: case 12: return skip(8);
            case 8: {
                const uint64_t len = get<uint64_t>();
                return ok && skip(len);
            }
            case 9: {
                if (depth > 16) return ok = false;
                const uint32_t et = get<uint32_t>();
                const uint64_t n = get<uint64_t>();
                for (uint64_t i = 0; ok && i < n; ++i) skip_value((int)et, depth + 1);
                return ok;
            }
            default:
                return ok = false;
        }
    }
};

int scalar_size(int t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

int parse(jinf_hip_gguf* g, FILE* f) {
    Reader r{f};
    const uint32_t magic = r.get<uint32_t>();
    if (!r.ok || magic != kGgufMagic) {
        JINF_LOG("Invalid GGUF magic: 0x%08X (expected 0x%08X)", magic, kGgufMagic);
        return JINF_HIP_ERR_PARSE;
    }
    g->version = r.get<uint32_t>();
    if (!r.ok || (g->version != 2 && g->version != 3)) {
        JINF_LOG("Unsupported GGUF version: %u", g->version);
        return JINF_HIP_ERR_PARSE;
    }
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    if (!r.ok) return JINF_HIP_ERR_PARSE;
    // every entry takes at least 12 bytes: a count past the file is malformed
    if (n_kv > g->file_size / 12 || n_tensors > g->file_size / 12) return JINF_HIP_ERR_PARSE;

    g->kvs.resize(n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        jinf_hip_gguf::KV& kv = g->kvs[i];
        if (!r.string(kv.key)) return JINF_HIP_ERR_PARSE;
        kv.type = (int)r.get<uint32_t>();
        if (!r.ok) return JINF_HIP_ERR_PARSE;
        const int sz = scalar_size(kv.type);
        if (sz) {
            if (fread(&kv.raw, (size_t)sz, 1, f) != 1) return JINF_HIP_ERR_PARSE;
        } else if (kv.type == 8) {
            if (!r.string(kv.str)) return JINF_HIP_ERR_PARSE;
        } else if (kv.type == 9) {
            kv.elem_type = (int)r.get<uint32_t>();
            kv.count = r.get<uint64_t>();
            for (uint64_t e = 0; r.ok && e < kv.count; ++e) r.skip_value(kv.elem_type);
            if (!r.ok) return JINF_HIP_ERR_PARSE;
        } else {
            return JINF_HIP_ERR_PARSE;
        }
        if (kv.key == "general.alignment" && kv.type == 4) g->alignment = (uint32_t)kv.raw;
    }
    if (g->alignment == 0) return JINF_HIP_ERR_PARSE;

    g->names.resize(n_tensors);
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        jinf_hip_gguf_tensor& t = g->tensors[i];
        memset(&t, 0, sizeof(t));
        if (!r.string(g->names[i])) return JINF_HIP_ERR_PARSE;
        t.n_dims = r.get<uint32_t>();
        if (!r.ok || t.n_dims > 4) return JINF_HIP_ERR_PARSE;
        // shape product and byte size with overflow checks: a negative
        // dimension or a product past int64 is a malformed file
        t.n_elements = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            t.shape[d] = r.get<int64_t>();
            if (t.shape[d] < 0 || __builtin_mul_overflow(t.n_elements, t.shape[d], &t.n_elements))
                return JINF_HIP_ERR_PARSE;
        }
        t.qtype = map_type(r.get<uint32_t>());
        t.offset = r.get<uint64_t>();
        if (!r.ok) return JINF_HIP_ERR_PARSE;
        int block, bytes;
        type_geometry(t.qtype, &block, &bytes);
        t.n_bytes = 0;
        if (block) {
            const uint64_t blocks = ((uint64_t)t.n_elements + (uint64_t)block - 1) / (uint64_t)block;
            if (__builtin_mul_overflow(blocks, (uint64_t)bytes, &t.n_bytes)) return JINF_HIP_ERR_PARSE;
        }
    }
    const uint64_t pos = (uint64_t)ftello(f);
    g->data_offset = (pos + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_offset < pos || g->data_offset > g->file_size) return JINF_HIP_ERR_PARSE;
    const uint64_t data_bytes = g->file_size - g->data_offset;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        g->tensors[i].name = g->names[i].c_str();
        const jinf_hip_gguf_tensor& t = g->tensors[i];
        // data_offset + offset + n_bytes <= file_size, written so nothing wraps
        if (t.offset > data_bytes || t.n_bytes > data_bytes - t.offset) return JINF_HIP_ERR_PARSE;
    }
    return JINF_HIP_OK;
}

void fill_hparams(jinf_hip_gguf* g) {
    jinf_hip_gguf_hparams& hp = g->hp;
    memset(&hp, 0, sizeof(hp));
    const char* arch = jinf_hip_gguf_get_str(g, "general.architecture", "llama");
    strncpy(hp.arch, arch, sizeof(hp.arch) - 1);
    const std::string pre = std::string(hp.arch) + ".";
    auto u32 = [&](const char* k, uint32_t def) {
        return jinf_hip_gguf_get_u32(g, (pre + k).c_str(), def);
    };
    auto f32 = [&](const char* k, float def) {
        return jinf_hip_gguf_get_f32(g, (pre + k).c_str(), def);
    };
    hp.n_layers = u32("block_count", 0);
    hp.n_embd = u32("embedding_length", 0);
    hp.n_heads = u32("attention.head_count", 0);
    hp.n_heads_kv = u32("attention.head_count_kv", 0);
    hp.n_ff = u32("feed_forward_length", 0);
    hp.n_vocab = u32("vocab_size", 0);
    hp.n_ctx_train = u32("context_length", 2048);
    hp.rope_freq_base = f32("rope.freq_base", 10000.0f);
    hp.rms_norm_eps = f32("attention.layer_norm_rms_epsilon", 1e-5f);
    if (hp.n_heads_kv == 0) hp.n_heads_kv = hp.n_heads;
    if (hp.n_vocab == 0) {
        const int64_t e = jinf_hip_gguf_find_tensor(g, "token_embd.weight");
        if (e >= 0 && g->tensors[e].n_dims >= 2) hp.n_vocab = (uint32_t)g->tensors[e].shape[1];
    }
}

// One lane per 18-byte block: upstream order (element j in the low nibble of
// qs[j], element j + 16 in its high nibble) -> jinf order (elements 2i, 2i+1
// in the low and high nibble of qs[i]).
__global__ __launch_bounds__(256) void q4_0_repack_kernel(uint8_t* __restrict__ blocks,
                                                          int64_t n_blocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    uint8_t* qs = blocks + 18 * b + 2;
    uint8_t in[16], out[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) in[j] = qs[j];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        out[i] = (uint8_t)((in[2 * i] & 0x0F) | ((in[2 * i + 1] & 0x0F) << 4));
        out[8 + i] = (uint8_t)((in[2 * i] >> 4) | (in[2 * i + 1] & 0xF0));
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) qs[j] = out[j];
}

}  // namespace
}  // namespace jinf


extern "C" int jinf_hip_gguf_load(jinf_hip_gguf** out, const char* path) {
    if (!out || !path) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) {
        JINF_LOG("Failed to open %s: %s", path, strerror(errno));
        return JINF_HIP_ERR_IO;
    }
    jinf_hip_gguf* g = new (std::nothrow) jinf_hip_gguf;
    if (!g) {
        fclose(f);
        return JINF_HIP_ERR_OOM;
    }
    g->path = path;
    struct stat st;
    g->file_size = fstat(fileno(f), &st) == 0 ? (uint64_t)st.st_size : 0;
    int rc;
    try {
        rc = jinf::parse(g, f);
    } catch (const std::bad_alloc&) {
        rc = JINF_HIP_ERR_OOM;
    }
    fclose(f);
    if (rc != JINF_HIP_OK) {
        delete g;
        return rc;
    }
    jinf::fill_hparams(g);
    *out = g;
    return JINF_HIP_OK;
}

extern "C" void jinf_hip_gguf_free(jinf_hip_gguf* g) { delete g; }

extern "C" uint32_t jinf_hip_gguf_version(const jinf_hip_gguf* g) { return g ? g->version : 0; }
extern "C" uint32_t jinf_hip_gguf_alignment(const jinf_hip_gguf* g) { return g ? g->alignment : 0; }
extern "C" uint64_t jinf_hip_gguf_data_offset(const jinf_hip_gguf* g) { return g ? g->data_offset : 0; }
extern "C" uint64_t jinf_hip_gguf_n_kv(const jinf_hip_gguf* g) { return g ? g->kvs.size() : 0; }
extern "C" uint64_t jinf_hip_gguf_n_tensors(const jinf_hip_gguf* g) { return g ? g->tensors.size() : 0; }

extern "C" const jinf_hip_gguf_hparams* jinf_hip_gguf_hparams_of(const jinf_hip_gguf* g) {
    return g ? &g->hp : nullptr;
}

extern "C" int64_t jinf_hip_gguf_find_kv(const jinf_hip_gguf* g, const char* key) {
    if (!g || !key) return -1;
    for (size_t i = 0; i < g->kvs.size(); ++i)
        if (g->kvs[i].key == key) return (int64_t)i;
    return -1;
}

extern "C" const char* jinf_hip_gguf_kv_key(const jinf_hip_gguf* g, uint64_t i) {
    return g && i < g->kvs.size() ? g->kvs[i].key.c_str() : nullptr;
}

extern "C" int jinf_hip_gguf_kv_type(const jinf_hip_gguf* g, uint64_t i) {
    return g && i < g->kvs.size() ? g->kvs[i].type : -1;
}

extern "C" int jinf_hip_gguf_kv_scalar(const jinf_hip_gguf* g, uint64_t i, void* out) {
    if (!g || i >= g->kvs.size() || !out) return JINF_HIP_ERR_INVALID;
    const int sz = jinf::scalar_size(g->kvs[i].type);
    if (!sz) return JINF_HIP_ERR_INVALID;
    memcpy(out, &g->kvs[i].raw, (size_t)sz);
    return JINF_HIP_OK;
}

extern "C" const char* jinf_hip_gguf_kv_str(const jinf_hip_gguf* g, uint64_t i) {
    return g && i < g->kvs.size() && g->kvs[i].type == 8 ? g->kvs[i].str.c_str() : nullptr;
}

extern "C" int jinf_hip_gguf_kv_array(const jinf_hip_gguf* g, uint64_t i, int* elem_type,
                                      uint64_t* count) {
    if (!g || i >= g->kvs.size() || g->kvs[i].type != 9) return JINF_HIP_ERR_INVALID;
    if (elem_type) *elem_type = g->kvs[i].elem_type;
    if (count) *count = g->kvs[i].count;
    return JINF_HIP_OK;
}

// Typed getters with the reference's conversions (src/gguf.cpp:343-381).
extern "C" const char* jinf_hip_gguf_get_str(const jinf_hip_gguf* g, const char* key,
                                             const char* def) {
    const int64_t i = jinf_hip_gguf_find_kv(g, key);
    return i >= 0 && g->kvs[i].type == 8 ? g->kvs[i].str.c_str() : def;
}

extern "C" uint32_t jinf_hip_gguf_get_u32(const jinf_hip_gguf* g, const char* key, uint32_t def) {
    const int64_t i = jinf_hip_gguf_find_kv(g, key);
    if (i < 0) return def;
    const jinf_hip_gguf::KV& kv = g->kvs[i];
    switch (kv.type) {
        case 4: return (uint32_t)kv.raw;
        case 5: { int32_t v; memcpy(&v, &kv.raw, 4); return (uint32_t)v; }
        case 10: return (uint32_t)kv.raw;
        case 11: { int64_t v; memcpy(&v, &kv.raw, 8); return (uint32_t)v; }
        case 6: { float v; memcpy(&v, &kv.raw, 4); return (uint32_t)v; }
        default: return def;
    }
}

extern "C" float jinf_hip_gguf_get_f32(const jinf_hip_gguf* g, const char* key, float def) {
    const int64_t i = jinf_hip_gguf_find_kv(g, key);
    if (i < 0) return def;
    const jinf_hip_gguf::KV& kv = g->kvs[i];
    switch (kv.type) {
        case 6: { float v; memcpy(&v, &kv.raw, 4); return v; }
        case 12: { double v; memcpy(&v, &kv.raw, 8); return (float)v; }
        case 4: return (float)(uint32_t)kv.raw;
        case 5: { int32_t v; memcpy(&v, &kv.raw, 4); return (float)v; }
        default: return def;
    }
}

extern "C" int64_t jinf_hip_gguf_find_tensor(const jinf_hip_gguf* g, const char* name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->names.size(); ++i)
        if (g->names[i] == name) return (int64_t)i;
    return -1;
}

extern "C" const jinf_hip_gguf_tensor* jinf_hip_gguf_tensor_at(const jinf_hip_gguf* g,
                                                               uint64_t i) {
    return g && i < g->tensors.size() ? &g->tensors[i] : nullptr;
}

extern "C" int jinf_hip_gguf_upload(const jinf_hip_gguf* g, uint64_t i, void* dst,
                                    uint64_t dst_bytes, hipStream_t stream) {
    if (!g || i >= g->tensors.size() || !dst) return JINF_HIP_ERR_INVALID;
    const jinf_hip_gguf_tensor& t = g->tensors[i];
    if (dst_bytes < t.n_bytes) return JINF_HIP_ERR_INVALID;
    return jinf::upload_file_range(g->path.c_str(), g->data_offset + t.offset, t.n_bytes, dst,
                                   stream);
}

extern "C" int jinf_hip_q4_0_repack_ggml(void* blocks, int64_t n_blocks, hipStream_t stream) {
    if (n_blocks < 0 || (n_blocks > 0 && !blocks)) return JINF_HIP_ERR_INVALID;
    if (n_blocks == 0) return JINF_HIP_OK;
    const int64_t grid = (n_blocks + 255) / 256;
    if (grid > 0x7FFFFFFF) return JINF_HIP_ERR_INVALID;
    return jinf::launch(jinf::q4_0_repack_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                        static_cast<uint8_t*>(blocks), n_blocks);
}
