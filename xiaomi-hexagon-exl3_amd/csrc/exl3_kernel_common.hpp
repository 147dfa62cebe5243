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

// Split-K hand-off through L2, without cache maintenance.  The partial sums of
// a column group's k-splits cross XCDs (each XCD has its own L2): they are
// written and read as 64-bit relaxed atomics at agent scope (sc1: coherent at
// device scope), each value tagged with the column group's generation number.
// Every workgroup bumps the group's arrival counter; the one that sees the
// last count sums the partials, re-reading (boundedly) any word whose tag is
// not yet the current generation, then advances the generation and clears the
// counter for the next call.  Correctness rests only on the coherence of each
// 64-bit word, so no release/acquire fence is needed; an agent-scope fence
// would write back and invalidate the whole L2 on gfx950 (measured 14.6 ->
// 53.8 us per call at k = 14336, n = 4096).  Waiting for the partial stores
// before the counter bump keeps re-reads from happening in practice.
constexpr int kTagSpinLimit = 1 << 20;

__device__ __forceinline__ unsigned load_relaxed(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_relaxed(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_tagged(uint64_t *p, float v, unsigned gen) {
    __hip_atomic_store(p, (uint64_t)__float_as_uint(v) | (uint64_t)gen << 32, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_tagged(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// the value of word p (first read w) once its tag is gen; NaN if it never
// becomes so within kTagSpinLimit re-reads (a loud result, never a hang)
__device__ __forceinline__ float tagged_value(const uint64_t *p, uint64_t w, unsigned gen) {
    if ((unsigned)(w >> 32) != gen) {
        int spin = 0;
        do {
            __builtin_amdgcn_s_sleep(1);
            w = load_tagged(p);
        } while ((unsigned)(w >> 32) != gen && ++spin < kTagSpinLimit);
        if ((unsigned)(w >> 32) != gen) return __builtin_nanf("");
    }
    return __uint_as_float((uint32_t)w);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// true in every thread of the last of `total` arriving workgroups
__device__ __forceinline__ bool arrive_last(unsigned *counter, unsigned total, int *flag_lds) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        *flag_lds = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    return *flag_lds != 0;
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
