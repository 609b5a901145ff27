// File-to-device copies shared by the model-file readers (GGUF, NVMW).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jinf {

// Copies n_bytes of the file at `path` starting at byte `offset` into device
// memory at dst, through two 32 MiB pinned staging buffers: the file read of
// chunk k + 1 overlaps the host-to-device copy of chunk k on `stream`.  A
// loader call: it allocates and frees the staging buffers and returns after
// the stream has finished the copies.  Status: 0 OK, 1 I/O (open, short
// read), 3 device.
int upload_file_range(const char* path, uint64_t offset, uint64_t n_bytes, void* dst,
                      hipStream_t stream);

}  // namespace jinf
