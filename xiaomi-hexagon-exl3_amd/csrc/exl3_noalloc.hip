// exl3_noalloc.hip -- exl3_hip_mul_mat_noalloc: the layer for callers that cannot
// allocate (code under HIP-graph capture, serving loops that forbid hipMalloc).
// Its workspace is the file-scope device array `scratch` below, one copy per GPU,
// of kNoallocScratchBytes; the GPU holds it until the process ends.  The array's
// device address is looked up once per device (hipGetSymbolAddress) and only
// that address is handed to kernels and fills; the name `scratch` itself is a
// host-side stand-in in host code.
#include <hip/hip_runtime.h>

#include <mutex>

#include "exl3_hip.h"
#include "exl3_launch.hpp"

namespace {

constexpr size_t kNoallocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, or null

// The current device's scratch address.  On a device's first call the array's
// split-K exchange is cleared on `stream` with a fill kernel (no hipMemsetAsync,
// so a first call under capture stays replay-safe); every later call finds it
// zero again because each GEMV call leaves it so.
exl3_status scratch_of_current_device(hipStream_t stream, void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return EXL3_HIP_ERROR;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return EXL3_HIP_ERROR;
        if (exl3k::launch_zero(p, exl3k::kSharedPrefixBytes, stream) != hipSuccess) return EXL3_HIP_ERROR;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return EXL3_OK;
}

}  // namespace

extern "C" exl3_status exl3_hip_mul_mat_noalloc(const void *records, unsigned bits, unsigned codebook, size_t k,
                                                size_t n, const void *x, exl3_dtype xt, size_t rows,
                                                size_t x_row_stride, void *y, exl3_dtype yt, size_t y_row_stride,
                                                hipStream_t stream) {
    if (!exl3_hip_supports_mul_mat(bits, codebook, k, n, rows, xt, yt)) return EXL3_INVAL_PARAMS;
    // workspaces beyond the array are refused before anything is enqueued
    if (exl3_hip_mul_mat_workspace_bytes(k, n, rows) > kNoallocScratchBytes) return EXL3_WORKSPACE_TOO_SMALL;
    void *ws = nullptr;
    const exl3_status st = scratch_of_current_device(stream, &ws);
    if (st != EXL3_OK) return st;
    return exl3_hip_mul_mat(records, bits, codebook, k, n, x, xt, rows, x_row_stride, y, yt, y_row_stride, ws,
                            kNoallocScratchBytes, stream);
}
