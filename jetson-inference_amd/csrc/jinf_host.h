// Host-side helpers for the jinf C-ABI launchers: status codes, argument
// checks and a kernel launch that reports the launch error directly
// (hipLaunchKernel's return value) instead of reading the thread's sticky
// last-error slot, which other libraries in the process may have set.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <tuple>
#include <utility>

#include "jinf/kernels_ext.h"

#define JINF_LOG(fmt, ...) fprintf(stderr, "[jinf] " fmt "\n", ##__VA_ARGS__)

namespace jinf {

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

template <typename Tuple, size_t... I>
inline int launch_impl(const void* fn, dim3 grid, dim3 block, size_t shmem,
                       hipStream_t stream, Tuple& args, std::index_sequence<I...>) {
    void* ptrs[sizeof...(I) + 1] = {(void*)&std::get<I>(args)..., nullptr};
    const hipError_t e = hipLaunchKernel(fn, grid, block, ptrs, shmem, stream);
    if (e != hipSuccess) {
        JINF_LOG("kernel launch failed: %s", hipGetErrorString(e));
        return JINF_HIP_ERR_DEVICE;
    }
    return JINF_HIP_OK;
}

// Launch `kern` with arguments converted to the kernel's exact parameter types.
template <typename... KArgs, typename... Args>
inline int launch(void (*kern)(KArgs...), dim3 grid, dim3 block, size_t shmem,
                  hipStream_t stream, Args... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    std::tuple<KArgs...> t(static_cast<KArgs>(args)...);
    return launch_impl(reinterpret_cast<const void*>(kern), grid, block, shmem, stream, t,
                       std::index_sequence_for<KArgs...>{});
}

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

}  // namespace jinf
