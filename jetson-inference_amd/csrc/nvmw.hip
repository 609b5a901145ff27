// .nvmw model files (the container jinf's prepare_model tool writes and its
// engine loads): header, layer index and tensor index parse, tensor upload
// into HBM.
//
// The on-disk structures are the reference's packed header and naturally
// aligned index records (include/jinf/nvmw.h:24-100); they are decoded here
// field by field at fixed little-endian byte offsets, so the layout does not
// depend on this compiler's struct packing:
//   header (4096 B): magic 0, version 4, n_layers 8, n_tensors 12,
//     index_offset 16, index_size 24, hot_offset 32, hot_size 40,
//     cold_start_offset 48, cold_total_size 56, n_embd 64, n_heads 68,
//     n_heads_kv 72, n_ff 76, n_vocab 80, n_ctx_train 84, rope_freq_base 88,
//     rms_norm_eps 92, primary_type 96, bundle_index_offset 104;
//   layer descriptor (24 B): cold_start_offset 0, cold_total_size 8,
//     n_cold_tensors 16;
//   tensor entry (200 B): name[128] 0, type 128, shape[4] 136, n_dims 168,
//     offset 176, n_bytes 184, layer_index 192, is_hot 196;
//   bundle header (16 B, packed): n_bundle_layers 0, bundle_size 4, n_ff 8;
//     then per layer (24 B, packed): bundles_offset 0, total 8, n_neurons 16,
//     bundle_size 20.
// Like the reference reader (src/nvmw.cpp:194-259) only the magic is
// checked, not the version, and a bundle index that cannot be read leaves
// the file without bundles.  Unlike it, an index or tensor data past the end
// of the file, and a cold tensor whose layer has no descriptor, are parse
// errors (the reference would read past its buffers later).
#include <errno.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <new>
#include <string>
#include <vector>

#include "file_io.h"
#include "jinf_host.h"
#include "jinf/nvmw_hip.h"

struct jinf_hip_nvmw {
    std::string path;
    uint64_t file_size = 0;
    jinf_hip_nvmw_header hdr{};
    std::vector<uint64_t> cold_start, cold_size;
    std::vector<std::string> names;
    std::vector<jinf_hip_nvmw_tensor> tensors;
    bool has_bundles = false;
};

namespace jinf {
namespace {

constexpr uint32_t kNvmwMagic = 0x574D564Eu;  // "NVMW" little-endian
constexpr size_t kHeaderBytes = 4096, kLayerBytes = 24, kEntryBytes = 200;
constexpr size_t kBundleHeaderBytes = 16, kBundleLayerBytes = 24;

template <typename T>
T rd(const uint8_t* p) {
    T v;
    memcpy(&v, p, sizeof v);
    return v;
}

bool read_at(FILE* f, uint64_t off, void* dst, size_t n) {
    return fseeko(f, (off_t)off, SEEK_SET) == 0 && fread(dst, 1, n, f) == n;
}

int parse(jinf_hip_nvmw* m, FILE* f) {
    uint8_t h[kHeaderBytes];
    if (m->file_size < kHeaderBytes || !read_at(f, 0, h, sizeof h)) return JINF_HIP_ERR_PARSE;
    jinf_hip_nvmw_header& H = m->hdr;
    H.magic = rd<uint32_t>(h + 0);
    if (H.magic != kNvmwMagic) {
        JINF_LOG("Invalid NVMW magic: 0x%08X", H.magic);
        return JINF_HIP_ERR_PARSE;
    }
    H.version = rd<uint32_t>(h + 4);
    H.n_layers = rd<uint32_t>(h + 8);
    H.n_tensors = rd<uint32_t>(h + 12);
    H.index_offset = rd<uint64_t>(h + 16);
    H.index_size = rd<uint64_t>(h + 24);
    H.hot_offset = rd<uint64_t>(h + 32);
    H.hot_size = rd<uint64_t>(h + 40);
    H.cold_start_offset = rd<uint64_t>(h + 48);
    H.cold_total_size = rd<uint64_t>(h + 56);
    H.n_embd = rd<uint32_t>(h + 64);
    H.n_heads = rd<uint32_t>(h + 68);
    H.n_heads_kv = rd<uint32_t>(h + 72);
    H.n_ff = rd<uint32_t>(h + 76);
    H.n_vocab = rd<uint32_t>(h + 80);
    H.n_ctx_train = rd<uint32_t>(h + 84);
    H.rope_freq_base = rd<float>(h + 88);
    H.rms_norm_eps = rd<float>(h + 92);
    H.primary_type = rd<int32_t>(h + 96);
    H.bundle_index_offset = rd<uint64_t>(h + 104);

    // the index must lie inside the file
    const uint64_t idx_bytes = (uint64_t)H.n_layers * kLayerBytes + (uint64_t)H.n_tensors * kEntryBytes;
    if (H.index_offset > m->file_size || idx_bytes > m->file_size - H.index_offset) {
        JINF_LOG("NVMW index past the end of the file");
        return JINF_HIP_ERR_PARSE;
    }
    std::vector<uint8_t> idx((size_t)idx_bytes);
    if (idx_bytes && !read_at(f, H.index_offset, idx.data(), idx.size())) return JINF_HIP_ERR_PARSE;
    m->cold_start.resize(H.n_layers);
    m->cold_size.resize(H.n_layers);
    for (uint32_t L = 0; L < H.n_layers; ++L) {
        const uint8_t* p = idx.data() + (size_t)L * kLayerBytes;
        m->cold_start[L] = rd<uint64_t>(p);
        m->cold_size[L] = rd<uint64_t>(p + 8);
    }
    m->names.resize(H.n_tensors);
    m->tensors.resize(H.n_tensors);
    for (uint32_t i = 0; i < H.n_tensors; ++i) {
        const uint8_t* p = idx.data() + (size_t)H.n_layers * kLayerBytes + (size_t)i * kEntryBytes;
        m->names[i].assign(reinterpret_cast<const char*>(p), strnlen(reinterpret_cast<const char*>(p), 128));
        jinf_hip_nvmw_tensor& t = m->tensors[i];
        t.qtype = rd<int32_t>(p + 128);
        for (int d = 0; d < 4; ++d) t.shape[d] = rd<int64_t>(p + 136 + 8 * d);
        t.n_dims = rd<uint32_t>(p + 168);
        t.offset = rd<uint64_t>(p + 176);
        t.n_bytes = rd<uint64_t>(p + 184);
        t.layer_index = rd<int32_t>(p + 192);
        t.is_hot = p[196] != 0;
        uint64_t base;
        if (t.is_hot) {
            base = H.hot_offset;
        } else if (t.layer_index >= 0 && (uint32_t)t.layer_index < H.n_layers) {
            base = m->cold_start[t.layer_index];
        } else {
            JINF_LOG("NVMW tensor %s: cold, layer %d has no descriptor", m->names[i].c_str(),
                     t.layer_index);
            return JINF_HIP_ERR_PARSE;
        }
        t.file_offset = base + t.offset;
        if (t.file_offset < base || t.file_offset > m->file_size ||
            t.n_bytes > m->file_size - t.file_offset) {
            JINF_LOG("NVMW tensor %s: data past the end of the file", m->names[i].c_str());
            return JINF_HIP_ERR_PARSE;
        }
    }
    for (uint32_t i = 0; i < H.n_tensors; ++i) m->tensors[i].name = m->names[i].c_str();

    // the sparse-FFN bundle index, when present and readable
    if (H.bundle_index_offset != 0) {
        uint8_t bh[kBundleHeaderBytes];
        if (read_at(f, H.bundle_index_offset, bh, sizeof bh)) {
            const uint32_t nl = rd<uint32_t>(bh);
            const uint64_t need = (uint64_t)nl * kBundleLayerBytes;
            std::vector<uint8_t> bl(need);
            m->has_bundles = need <= m->file_size &&
                             (need == 0 || read_at(f, H.bundle_index_offset + sizeof bh,
                                                   bl.data(), bl.size()));
        }
    }
    return JINF_HIP_OK;
}

}  // namespace
}  // namespace jinf

extern "C" int jinf_hip_nvmw_load(jinf_hip_nvmw** out, const char* path) {
    if (!out || !path) return JINF_HIP_ERR_INVALID;
    *out = nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) {
        JINF_LOG("Failed to open %s: %s", path, strerror(errno));
        return JINF_HIP_ERR_IO;
    }
    jinf_hip_nvmw* m = new (std::nothrow) jinf_hip_nvmw;
    if (!m) {
        fclose(f);
        return JINF_HIP_ERR_OOM;
    }
    m->path = path;
    struct stat st;
    m->file_size = fstat(fileno(f), &st) == 0 ? (uint64_t)st.st_size : 0;
    int rc;
    try {
        rc = jinf::parse(m, f);
    } catch (const std::bad_alloc&) {
        rc = JINF_HIP_ERR_OOM;
    }
    fclose(f);
    if (rc != JINF_HIP_OK) {
        delete m;
        return rc;
    }
    *out = m;
    return JINF_HIP_OK;
}

extern "C" void jinf_hip_nvmw_free(jinf_hip_nvmw* m) { delete m; }

extern "C" const jinf_hip_nvmw_header* jinf_hip_nvmw_header_of(const jinf_hip_nvmw* m) {
    return m ? &m->hdr : nullptr;
}

extern "C" uint64_t jinf_hip_nvmw_n_tensors(const jinf_hip_nvmw* m) {
    return m ? m->tensors.size() : 0;
}

extern "C" const jinf_hip_nvmw_tensor* jinf_hip_nvmw_tensor_at(const jinf_hip_nvmw* m, uint64_t i) {
    return m && i < m->tensors.size() ? &m->tensors[i] : nullptr;
}

extern "C" int64_t jinf_hip_nvmw_find_tensor(const jinf_hip_nvmw* m, const char* name) {
    if (!m || !name) return -1;
    for (size_t i = 0; i < m->names.size(); ++i)
        if (m->names[i] == name) return (int64_t)i;
    return -1;
}

extern "C" int jinf_hip_nvmw_layer_cold_range(const jinf_hip_nvmw* m, int layer, uint64_t* offset,
                                              uint64_t* size) {
    if (!m || !offset || !size || layer < 0 || (size_t)layer >= m->cold_start.size())
        return JINF_HIP_ERR_INVALID;
    *offset = m->cold_start[layer];
    *size = m->cold_size[layer];
    return JINF_HIP_OK;
}

extern "C" int jinf_hip_nvmw_has_bundles(const jinf_hip_nvmw* m) { return m && m->has_bundles; }

extern "C" int jinf_hip_nvmw_upload(const jinf_hip_nvmw* m, uint64_t i, void* dst,
                                    uint64_t dst_bytes, hipStream_t stream) {
    if (!m || i >= m->tensors.size() || !dst) return JINF_HIP_ERR_INVALID;
    const jinf_hip_nvmw_tensor& t = m->tensors[i];
    if (dst_bytes < t.n_bytes) return JINF_HIP_ERR_INVALID;
    return jinf::upload_file_range(m->path.c_str(), t.file_offset, t.n_bytes, dst, stream);
}
