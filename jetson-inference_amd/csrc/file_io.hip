// File-to-device copies through pinned staging buffers (see file_io.h).
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <unistd.h>

#include "file_io.h"
#include "jinf_host.h"

namespace jinf {

int upload_file_range(const char* path, uint64_t offset, uint64_t n_bytes, void* dst,
                      hipStream_t stream) {
    if (n_bytes == 0) return JINF_HIP_OK;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        JINF_LOG("Failed to open %s: %s", path, strerror(errno));
        return JINF_HIP_ERR_IO;
    }
    constexpr size_t kChunk = 32u << 20;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = JINF_HIP_OK;
    for (int b = 0; b < 2 && rc == JINF_HIP_OK; ++b) {
        if (hipHostMalloc(&stage[b], kChunk, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess)
            rc = JINF_HIP_ERR_DEVICE;
    }
    for (uint64_t off = 0, k = 0; rc == JINF_HIP_OK && off < n_bytes; off += kChunk, ++k) {
        const int b = (int)(k & 1);
        const size_t n = (size_t)(n_bytes - off < kChunk ? n_bytes - off : kChunk);
        if (k >= 2 && hipEventSynchronize(done[b]) != hipSuccess) {  // buffer b free again
            rc = JINF_HIP_ERR_DEVICE;
            break;
        }
        size_t got = 0;
        while (got < n) {
            const ssize_t r = pread(fd, (char*)stage[b] + got, n - got, (off_t)(offset + off + got));
            if (r <= 0) break;
            got += (size_t)r;
        }
        if (got != n) {
            rc = JINF_HIP_ERR_IO;
            break;
        }
        if (hipMemcpyAsync((char*)dst + off, stage[b], n, hipMemcpyHostToDevice, stream) !=
                hipSuccess ||
            hipEventRecord(done[b], stream) != hipSuccess)
            rc = JINF_HIP_ERR_DEVICE;
    }
    // the staging buffers are released only after every copy from them ended
    if (hipStreamSynchronize(stream) != hipSuccess && rc == JINF_HIP_OK) rc = JINF_HIP_ERR_DEVICE;
    for (int b = 0; b < 2; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (stage[b]) (void)hipHostFree(stage[b]);
    }
    close(fd);
    return rc;
}

}  // namespace jinf
