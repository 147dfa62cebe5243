// exl3_kernel_common.hpp -- device helpers shared by the gfx950 kernel files
// (exl3_codec_kernels.hip, exl3_gemv.hip, exl3_gemm.hip): fp16 bit conversions,
// the record geometry, the split-K hand-off and the trellis word loads.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "exl3_device.hpp"
#include "exl3_launch.hpp"

namespace exl3k {

using namespace exl3dev;

__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return (float)bitcast<_Float16>(h); }
__device__ __forceinline__ uint16_t float_to_half_bits(float f) { return bitcast<uint16_t>((_Float16)f); }

__device__ __forceinline__ size_t group_bytes(int bits) { return (size_t)2048 * bits + 512; }

// Binary32 product rounded to binary32.  Kept opaque so the compiler cannot fuse
// a following fp16 conversion into one v_fma_mix rounding: the reference rounds
// to binary32 first and then to binary16 (src/exl3_codec.cpp:198-199).
__device__ __forceinline__ float mul_rn_f32(float a, float b) {
    float r;
    asm("v_mul_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Split-K partials cross XCDs (each XCD has its own L2).  They are written and
// read with agent-scope relaxed atomics (sc1: coherent at device scope, no L2
// write-back or invalidate of unrelated lines).  The hand-off is a release /
// acquire pair at agent scope: every thread's partial stores are ordered before
// the arrival counter's increment by an agent-scope release fence (each wave
// waits for its own stores) and the workgroup barrier, the increment itself is
// acq_rel, and the last workgroup's loads follow an agent-scope acquire fence.
__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// returns true in every thread of the last of `total` arriving workgroups; the
// partials of all earlier arrivals are then visible to it
__device__ __forceinline__ bool arrive_last(unsigned *counter, unsigned total, int *flag_lds) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0)
        *flag_lds = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    const bool last = *flag_lds != 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return last;
}
__device__ __forceinline__ void reset_counter(unsigned *counter) {
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tile address of trellis tile (rk, cn) of a k x n matrix.
template <int K>
__device__ __forceinline__ const uint32_t *tile_ptr(const uint8_t *src, int records_layout, size_t k, size_t n,
                                                    size_t rk, size_t cn) {
    if (records_layout) {
        const size_t nb = cn >> 3, kb = rk >> 3;
        const size_t off = (nb * (k >> 7) + kb) * group_bytes(K) + ((rk & 7) * 8 + (cn & 7)) * 32 * K;
        return (const uint32_t *)(src + off);
    }
    return (const uint32_t *)(src + (rk * (n >> 4) + cn) * 32 * K);
}

// ============================================================== activations
__device__ __forceinline__ float load_x(const void *x, int x_f16, size_t stride, size_t r, size_t i) {
    if (x_f16) return half_bits_to_float(((const uint16_t *)x)[r * stride + i]);
    return ((const float *)x)[r * stride + i];
}

// K contiguous words of a chunk, in as few loads as its alignment allows
template <int K>
__device__ __forceinline__ void load_chunk(const uint8_t *p, uint32_t (&w)[K]) {
    if constexpr (K % 4 == 0) {
#pragma unroll
        for (int v = 0; v < K / 4; ++v) {
            const u4 t = __builtin_nontemporal_load((const u4 *)p + v);
            w[4 * v] = t.x;
            w[4 * v + 1] = t.y;
            w[4 * v + 2] = t.z;
            w[4 * v + 3] = t.w;
        }
    } else if constexpr (K % 2 == 0) {
#pragma unroll
        for (int v = 0; v < K / 2; ++v) {
            const u2 t = __builtin_nontemporal_load((const u2 *)p + v);
            w[2 * v] = t.x;
            w[2 * v + 1] = t.y;
        }
    } else {
#pragma unroll
        for (int v = 0; v < K; ++v) w[v] = __builtin_nontemporal_load((const uint32_t *)p + v);
    }
}

}  // namespace exl3k
