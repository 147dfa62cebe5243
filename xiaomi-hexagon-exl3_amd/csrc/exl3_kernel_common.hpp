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
// a column group's k-splits cross XCDs (each XCD has its own L2), through the
// workspace's exchange: 32-bit words, zero ("empty") between calls.  Every
// workgroup but the column group's last split stores its partial there as
// relaxed agent-scope atomics (sc1: coherent at device scope), each value
// complemented and never zero (exchange_bits), and ends.  The last split's
// workgroup (the highest workgroup index of its column group) keeps its own
// partial in LDS, reads the other splits' words, reading again (in batches,
// boundedly) any word still empty, sums all splits in split order, then zeroes
// every word it read, so the next call finds the same state.  Within a call
// each word is zero or holds the value its one writer stored, and 32-bit words
// are single-copy atomic: a nonzero word is this call's value, whatever order
// the words arrive in.  That is why no release/acquire pair is needed; an
// agent-scope fence writes back or invalidates the whole L2 on gfx950 (measured
// 14.6 -> 53.8 us per GEMV call at k = 14336, n = 4096).  Only the summing
// workgroups wait, and only for workgroups that wait for nothing.  The split is
// the grid's slowest dimension, so the summing workgroups are the grid's last:
// on every XCD the others are dispatched before any of them and never need a
// slot that a waiting workgroup holds, and every wait ends.  Each wait is also
// bounded: a wave that has polled kExchangeSpinLimit times, or whose workgroup
// has already given up, stops waiting; the words still empty count as NaN and
// the workspace's status word (kStatusOffset) is set, which makes every later
// call with that workspace NaN until it is zero-filled again.
constexpr int kExchangeSpinLimit = 1 << 20;  // polls per wave of the summing workgroup before it gives up

// binary32 bits complemented; the one value whose complement is zero (the NaN
// 0xffffffff) is stored as 1, which reads back as the NaN 0xfffffffe
__device__ __forceinline__ uint32_t exchange_bits(float v) {
    const uint32_t c = ~__float_as_uint(v);
    return c ? c : 1u;
}
__device__ __forceinline__ float exchange_value(uint32_t w) { return __uint_as_float(~w); }
__device__ __forceinline__ void store_exchange(uint32_t *p, float v) {
    __hip_atomic_store(p, exchange_bits(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_exchange(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Empties four words (16-byte aligned) with one plain 16-byte store.  Only the
// summing workgroup clears, and only words it has already read full: each
// word's one store reached the device-coherent level before the agent-scope
// load that returned it, and nothing else writes or reads the word again in
// this call.  The zeros therefore land in this XCD's L2 after that store, and
// the write-back at the end of the kernel puts them in memory before the next
// call, which the stream orders after this one.  Relaxed agent-scope atomic
// stores, which write through to memory one word each, kept every summing
// workgroup alive until they were acknowledged: 0.3-0.8 us more per call.
// (In the language model the clear is not ordered after the writer's relaxed
// store, since reading a relaxed store creates no happens-before edge; the
// argument above is the hardware's.)
__device__ __forceinline__ void clear_exchange4(uint32_t *p) {
    *(uint4 *)p = make_uint4(0u, 0u, 0u, 0u);
}

// maximum of v over the wave, in every lane
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_xor<1>(v));
    v = fmaxf(v, dpp_xor<2>(v));
    v = fmaxf(v, dpp_xor<4>(v));
    v = fmaxf(v, dpp_xor<8>(v));
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
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
