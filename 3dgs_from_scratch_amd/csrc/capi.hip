// ABI-level helpers: status strings, version, and a kernel-based zero fill
// (used instead of hipMemsetAsync so that callers may capture every entry
// point into a HIP graph).

#include "gs_common.h"

namespace gs {

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *__restrict__ p, int64_t words) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride)
        p[i] = 0u;
}

__global__ void zero_tail_kernel(uint8_t *__restrict__ p, int64_t bytes) {
    const int64_t i = threadIdx.x;
    if (i < bytes) p[i] = 0;
}

int zero_bytes(void *ptr, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return GS_OK;
    if (!ptr) return GS_ERR_INVALID_ARGUMENT;
    const int64_t words = (int64_t)(bytes / 4);
    if (words > 0) {
        int64_t blocks = (words + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                           reinterpret_cast<uint32_t *>(ptr), words);
        const int st = launch_status();
        if (st) return st;
    }
    const int64_t tail = (int64_t)(bytes % 4);
    if (tail) {
        hipLaunchKernelGGL(zero_tail_kernel, dim3(1), dim3(4), 0, stream,
                           reinterpret_cast<uint8_t *>(ptr) + words * 4, tail);
        return launch_status();
    }
    return GS_OK;
}

}  // namespace gs

extern "C" const char *gs_status_string(int status) {
    switch (status) {
        case GS_OK:
            return "success";
        case GS_ERR_INVALID_ARGUMENT:
            return "invalid argument (negative size, null required pointer or bad tile size)";
        case GS_ERR_WORKSPACE_TOO_SMALL:
            return "workspace smaller than the size reported by the *_workspace_size query";
        case GS_ERR_TOO_MANY_KEYS:
            return "more than INT32_MAX (tile, Gaussian) intersections";
        case GS_ERR_UNSUPPORTED:
            return "unsupported argument combination (tile_size^2 must be <= 1024)";
        default:
            if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
            return "unknown status";
    }
}

extern "C" int gs_abi_version(void) { return 20; }

extern "C" int gs_host_device_pointer(void *host, void **device) {
    if (!host || !device) return GS_ERR_INVALID_ARGUMENT;
    *device = nullptr;
    const hipError_t e = hipHostGetDevicePointer(device, host, 0);
    if (e != hipSuccess) {
        *device = nullptr;
        return (int)e;
    }
    return *device ? GS_OK : GS_ERR_UNSUPPORTED;
}
